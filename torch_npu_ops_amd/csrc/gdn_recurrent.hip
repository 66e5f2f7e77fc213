// Gated delta rule, recurrent form (decode / short speculative windows),
// and the decode step fused with the causal conv1d update, for gfx950.
//
// Per token (reference kernel triton_npu/triton_src/
// test_fused_recurrent_gated_delta_rule.py:125-164, CPU golden
// triton_npu/test/triton_recurrent_gated_delta_rule_test.cpp:47-115):
//   q, k <- q/sqrt(sum q^2 + 1e-6), k/sqrt(sum k^2 + 1e-6)   (if l2norm)
//   q    <- q * scale
//   h    <- exp(g) * h                       h: [K, V] fp32 per (slot, head)
//   v'   <- beta * (v - h^T k)
//   h    <- h + k v'^T
//   o    <- h^T q
// GQA: v-head hv reads qk-head hv / (HV / H).  State slots come from
// ssm_state_indices; with num_accepted_tokens (speculative decoding) the
// initial state is column accepted-1 and the state after token t goes to
// column t (..._spec_fwd_kernel, :257-307).
//
// Design (HBM-bound state streaming): one 256-lane block per (sequence,
// v-head) keeps the whole K x V fp32 state in registers, K*V/256 values per
// lane laid out so that each row of V values is contiguous across V/4
// lanes (16-byte accesses, 1 KB per wave per instruction).  h^T k and h^T q
// of the decayed state come out of one pass over the registers and one
// cross-wave LDS reduction (o = (e^g h)^T q + (k.q) v', so the update and
// the output need no second pass); the rank-1 update is applied in
// registers and the state is written back once.  State traffic uses
// non-temporal hints: it is read and written exactly once per call.
#include "xk_common.h"

namespace xk {
namespace {

constexpr int kThreads = 256;
// The fused decode kernel keeps one block per (batch row, qk head) and
// spreads each 64 KB state tile over 512 lanes (8 loads per lane): an
// in-place stream of 64 KB tiles runs at 5.5 TB/s on MI355X with 16 loads
// per lane, at 6.2 TB/s with 8.
constexpr int kFusedThreads = 512;

// Per-lane share of a K x V state tile.
template <int K, int V, int NT = kThreads>
struct Tile {
  static constexpr int kLanesPerRow = V / 4;               // float4 per lane
  static constexpr int kRowsPerPass = NT / kLanesPerRow;
  static constexpr int kPasses = K / kRowsPerPass;
  static_assert(V % 4 == 0 && kLanesPerRow <= kWave && kWave % kLanesPerRow == 0,
                "row of V must fit a wave");
  static_assert(K % kRowsPerPass == 0, "K must be a multiple of rows per pass");
  float h[kPasses][4];
};

// LDS shared by one block: normalised q/k (fp32), v, the reduction scratch
// and the per-column results.
template <int K, int V, int NT = kThreads>
struct Smem {
  float q[K];
  float k[K];
  float v[V];
  float red[2][NT / kWave][V];  // per-wave partials of h^T k, h^T q
  float kh[V];
  float qh[V];
  float scal[4];  // k.q, ||q||^2, ||k||^2
};

template <typename T>
__device__ __forceinline__ float ldf(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const T*>(p)[i]);
}

// softplus(x) = max(x, 0) + log1p(e^-|x|) on the hardware exp2 / log2
// (v_exp_f32, v_log_f32).  e^-|x| = 2^p (1 + p_lo ln 2) with p = fl(-|x|
// log2 e) and p_lo its rounding error (one fma) plus the error of the
// float log2 e, so the result stays within a few ulp for large |x| too;
// log1p(u) = log(1 + u) * u / ((1 + u) - 1) (Goldberg's correction; (1 + u)
// - 1 is exact, and 1 + u == 1 gives u).  About 20 instructions against
// ~100 for log1pf(expf(x)).
__device__ __forceinline__ float softplus_hw(float x) {
  constexpr float kLog2e = 1.44269502162933349609375f;  // float(log2 e)
  constexpr float kLog2eLo = 1.925963e-08f;              // log2 e - kLog2e
  constexpr float kLn2 = 0.693147180559945309f;
  const float t = -fabsf(x);
  const float p = t * kLog2e;
  const float plo = fmaf(t, kLog2e, -p) + t * kLog2eLo;
  const float u0 = __builtin_amdgcn_exp2f(p);
  const float u = fmaf(u0, plo * kLn2, u0);
  const float w = 1.f + u;
  const float d = w - 1.f;
  const float lp = d == 0.f ? u : __builtin_amdgcn_logf(w) * kLn2 * (u * __builtin_amdgcn_rcpf(d));
  return fmaxf(x, 0.f) + lp;
}

// GDN gating (triton_src/test_fused_gdn_gating.py:30-43): the log-decay
// g = -exp(A_log) * softplus_{beta, threshold}(a + dt_bias), where softplus
// is log(1 + exp(beta x)) / beta below the threshold and x above it.  Both
// exponentials use the hardware exp2 (exp(A_log) to ~1e-7 |A_log|
// relative): g is fp32 and the reference's test holds it to rtol / atol
// 1e-3 (test_fused_gdn_gating.py:107); the error here is below 1e-6.
// inv_beta is 1 / sp_beta, multiplied in as the reference does.
__device__ __forceinline__ float gdn_log_decay(float a_plus_bias, float A_log, float sp_beta,
                                               float inv_beta, float threshold) {
  constexpr float kLog2e = 1.44269504088896341f;
  const float bx = sp_beta * a_plus_bias;
  const float sp = bx <= threshold ? inv_beta * softplus_hw(bx) : a_plus_bias;
  return -__builtin_amdgcn_exp2f(A_log * kLog2e) * sp;
}

// sigmoid with IEEE division and the accurate exp, so that a rounded
// 16-bit result matches a CPU computation of the same expression.
__device__ __forceinline__ float sigmoid_exact(float x) { return 1.0f / (1.0f + expf(-x)); }

// sigmoid(x) rounded to bf16, equal to sigmoid_exact's rounding.  For
// |x| < 32 the hardware exp2 / rcp value is within about 50 fp32 ulp of
// sigmoid_exact's: fl(-x log2 e) (< 64 in magnitude) is off by at most
// 2^-19 for its rounding plus 32 * 2^-24 for the float log2 e, i.e. 2^-18,
// which is 44 ulp of exp2 at most; exp2, the add, rcp and sigmoid_exact
// itself add a few more.  So when the fast value's low 16 bits are more than
// 128 from the bf16 rounding boundary 0x8000, both round to the same bf16.
// Elsewhere (0.4% of values, and |x| >= 32 or NaN) sigmoid_exact is used.
__device__ __forceinline__ bf16 sigmoid_bf16(float x) {
  constexpr float kLog2e = 1.44269504088896341f;
  float s = __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * kLog2e));
  const uint32_t low = __builtin_bit_cast(uint32_t, s) & 0xFFFFu;
  if (!(fabsf(x) < 32.f) || (low > 0x8000u - 128u && low < 0x8000u + 128u)) s = sigmoid_exact(x);
  return from_f32<bf16>(s);
}

template <typename AB>
__device__ __forceinline__ AB sigmoid_to(float x) {
  if constexpr (std::is_same<AB, bf16>::value) {
    return sigmoid_bf16(x);
  } else {
    return from_f32<AB>(sigmoid_exact(x));
  }
}

// One token of the recurrence on the register tile.  Inputs (q, k already
// normalised and q scaled) are in sm.q / sm.k / sm.v.  Writes o[V] through
// `out` (fp32 values, converted by the caller's store functor).
template <int K, int V, int NT, typename StoreO>
__device__ __forceinline__ void gdn_token(Tile<K, V, NT>& t, Smem<K, V, NT>& sm,
                                          float decay, float beta, StoreO store_o) {
  using TL = Tile<K, V, NT>;
  const int tid = threadIdx.x;
  const int c4 = tid % TL::kLanesPerRow;  // column group (4 columns)
  const int r0 = tid / TL::kLanesPerRow;  // first row
  const int wid = tid / kWave;
  __syncthreads();  // sm.q / sm.k / sm.v of this token are complete

  float pk[4] = {0.f, 0.f, 0.f, 0.f}, pq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < TL::kPasses; ++i) {
    const int r = r0 + i * TL::kRowsPerPass;
    const float kr = sm.k[r], qr = sm.q[r];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      t.h[i][c] *= decay;
      pk[c] = fmaf(t.h[i][c], kr, pk[c]);
      pq[c] = fmaf(t.h[i][c], qr, pq[c]);
    }
  }
  // Reduce over the rows held by the other lanes of this wave (same c4).
#pragma unroll
  for (int o = TL::kLanesPerRow; o < kWave; o <<= 1)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      pk[c] += __shfl_xor(pk[c], o, kWave);
      pq[c] += __shfl_xor(pq[c], o, kWave);
    }
  if ((tid % kWave) < TL::kLanesPerRow) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      sm.red[0][wid][c4 * 4 + c] = pk[c];
      sm.red[1][wid][c4 * 4 + c] = pq[c];
    }
  }
  __syncthreads();
  if (tid < V) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int w = 0; w < NT / kWave; ++w) {
      a += sm.red[0][w][tid];
      b += sm.red[1][w][tid];
    }
    // v' = beta (v - h^T k);  o = h^T q + (k.q) v'
    const float vn = beta * (sm.v[tid] - a);
    sm.kh[tid] = vn;
    store_o(tid, b + sm.scal[0] * vn);
  }
  __syncthreads();
  float vn[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) vn[c] = sm.kh[c4 * 4 + c];
#pragma unroll
  for (int i = 0; i < TL::kPasses; ++i) {
    const float kr = sm.k[r0 + i * TL::kRowsPerPass];
#pragma unroll
    for (int c = 0; c < 4; ++c) t.h[i][c] = fmaf(kr, vn[c], t.h[i][c]);
  }
}

template <int K, int V, int NT>
// `pitch`: floats between rows in memory (the tile may be a column slice of
// a wider state).
__device__ __forceinline__ void load_tile(Tile<K, V, NT>& t, const float* base, int64_t pitch = V) {
  using TL = Tile<K, V, NT>;
  const int c4 = threadIdx.x % TL::kLanesPerRow;
  const int r0 = threadIdx.x / TL::kLanesPerRow;
#pragma unroll
  for (int i = 0; i < TL::kPasses; ++i) {
    const Vec<float, 4> v = ld_stream(reinterpret_cast<const Vec<float, 4>*>(
        base + static_cast<int64_t>(r0 + i * TL::kRowsPerPass) * pitch + c4 * 4));
#pragma unroll
    for (int c = 0; c < 4; ++c) t.h[i][c] = v.v[c];
  }
}

template <int K, int V, int NT>
__device__ __forceinline__ void zero_tile(Tile<K, V, NT>& t) {
#pragma unroll
  for (int i = 0; i < Tile<K, V, NT>::kPasses; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) t.h[i][c] = 0.f;
}

template <int K, int V, int NT>
__device__ __forceinline__ void store_tile(const Tile<K, V, NT>& t, float* base, int64_t pitch = V) {
  using TL = Tile<K, V, NT>;
  const int c4 = threadIdx.x % TL::kLanesPerRow;
  const int r0 = threadIdx.x / TL::kLanesPerRow;
#pragma unroll
  for (int i = 0; i < TL::kPasses; ++i) {
    Vec<float, 4> v;
#pragma unroll
    for (int c = 0; c < 4; ++c) v.v[c] = t.h[i][c];
    st_stream(reinterpret_cast<Vec<float, 4>*>(
                  base + static_cast<int64_t>(r0 + i * TL::kRowsPerPass) * pitch + c4 * 4),
              v);
  }
}

// Loads q and k of one token (raw), then l2-normalises (optional) and
// scales q.  Block-wide; ends with a barrier.
template <int K, int V, int NT, typename LoadQK>
__device__ __forceinline__ void prep_qk(Smem<K, V, NT>& sm, LoadQK load, bool l2norm,
                                        float scale) {
  const int tid = threadIdx.x;
  // The previous token's readers of sm.q / sm.k / sm.scal are done.
  __syncthreads();
  if (tid < K) {
    const float qv = load(0, tid), kv = load(1, tid);
    sm.q[tid] = qv;
    sm.k[tid] = kv;
  }
  __syncthreads();
  if (tid < kWave) {
    float sq = 0.f, sk = 0.f, kq = 0.f;
    for (int i = tid; i < K; i += kWave) {
      sq = fmaf(sm.q[i], sm.q[i], sq);
      sk = fmaf(sm.k[i], sm.k[i], sk);
      kq = fmaf(sm.q[i], sm.k[i], kq);
    }
    sq = group_sum<kWave>(sq);
    sk = group_sum<kWave>(sk);
    kq = group_sum<kWave>(kq);
    if (tid == 0) {
      const float rq = l2norm ? 1.0f / sqrtf(sq + 1e-6f) : 1.0f;
      const float rk = l2norm ? 1.0f / sqrtf(sk + 1e-6f) : 1.0f;
      sm.scal[1] = rq * scale;
      sm.scal[2] = rk;
      sm.scal[0] = kq * rq * rk * scale;  // (k_hat . q_hat) * scale
    }
  }
  __syncthreads();
  if (tid < K) {
    sm.q[tid] *= sm.scal[1];
    sm.k[tid] *= sm.scal[2];
  }
  // sm.q / sm.k are read by other lanes in gdn_token after its first
  // barrier; sm.v must be written by the caller before that barrier too.
}

// ---------------------------------------------------------------------------
// Recurrent GDN over varlen sequences.
// ---------------------------------------------------------------------------
struct RecParams {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  void* o;
  const float* h0;
  float* ht;
  int64_t h0_slot_stride, ht_slot_stride;
  int64_t slots;  // rows of the state pool (valid slot range)
  const void* cu;
  int cu_i64;
  const int32_t* idx;
  int64_t idx_s0, idx_s1;
  const int32_t* accepted;
  int64_t N, T;  // sequences; tokens per sequence when cu == NULL
  int H, HV;
  float scale;
  int l2norm;
  int inplace;
  // Gating mode: g holds a and beta holds b ([tokens, HV]); per token
  // g = gdn_log_decay(a + dt_bias, A_log), beta = sigmoid(b).
  int gating;
  const float* A_log;
  const float* dt_bias;
  float sp_beta, sp_thr;
};

// NS blocks per (sequence, v head), each owning VT = V / NS state columns
// (the recurrence is independent per column; q / k normalisation is
// repeated per block).  At V = 128, NS = 2: an in-place stream of 64 KB
// tiles with 16 loads per lane runs at 5.5 TB/s on MI355X, of 32 KB tiles
// with 8 loads per lane at 6.3 TB/s.
template <int K, int V, typename T, typename GT, typename BT, int NS>
__global__ void __launch_bounds__(kThreads) gdn_recurrent_kernel(RecParams p) {
  constexpr int VT = V / NS;
  __shared__ Smem<K, VT> sm;
  const int cs = static_cast<int>(blockIdx.x % NS);  // column slice
  const int64_t item = blockIdx.x / NS;
  const int64_t n = item / p.HV;
  const int hv = static_cast<int>(item % p.HV);
  const int hq = hv / (p.HV / p.H);
  int64_t bos, len;
  if (p.cu) {
    const int64_t a = p.cu_i64 ? reinterpret_cast<const int64_t*>(p.cu)[n]
                               : reinterpret_cast<const int32_t*>(p.cu)[n];
    const int64_t b = p.cu_i64 ? reinterpret_cast<const int64_t*>(p.cu)[n + 1]
                               : reinterpret_cast<const int32_t*>(p.cu)[n + 1];
    bos = a;
    len = b - a;
  } else {
    bos = n * p.T;
    len = p.T;
  }
  if (len <= 0) return;  // whole block exits together

  const int64_t first_col = p.accepted ? p.accepted[n] - 1 : 0;
  auto slot_of = [&](int64_t col) -> int64_t {
    return p.idx ? p.idx[n * p.idx_s0 + col * p.idx_s1] : n;
  };
  // One token's inputs: lane tid holds element tid of q, k (tid < K) and v
  // (tid < V), plus the head's g and beta.
  const int tid = threadIdx.x;
  struct TokIn {
    float q, k, v, g, b;
  };
  auto load_in = [&](int64_t tok) {
    TokIn r;
    r.q = tid < K ? ldf<T>(p.q, (tok * p.H + hq) * K + tid) : 0.f;
    r.k = tid < K ? ldf<T>(p.k, (tok * p.H + hq) * K + tid) : 0.f;
    r.v = tid < VT ? ldf<T>(p.v, (tok * p.HV + hv) * V + cs * VT + tid) : 0.f;
    r.g = ldf<GT>(p.g, tok * p.HV + hv);
    r.b = p.beta ? ldf<BT>(p.beta, tok * p.HV + hv) : 1.0f;
    if (p.gating) {
      r.g = gdn_log_decay(r.g + p.dt_bias[hv], p.A_log[hv], p.sp_beta, 1.0f / p.sp_beta,
                          p.sp_thr);
      r.b = sigmoid_exact(r.b);
    }
    return r;
  };
  // The first token's inputs are fetched before the state tile: loads
  // complete in issue order, so the q/k normalisation then overlaps the
  // tile's latency instead of waiting behind it.
  TokIn cur = load_in(bos);
  Tile<K, VT> t;
  const int64_t s0 = slot_of(first_col);
  const bool s0_ok = p.h0 && s0 >= 0 && s0 < p.slots && first_col >= 0;
  const int64_t col0 = static_cast<int64_t>(hv) * K * V + cs * VT;  // slice within a slot
  if (s0_ok)
    load_tile<K, VT>(t, p.h0 + s0 * p.h0_slot_stride + col0, V);
  else
    zero_tile<K, VT>(t);

  // Per-token state writes: in place with a per-token slot column (2-D
  // indices or speculative decoding); otherwise once at the end.
  const bool per_token = p.inplace && p.idx && p.idx_s1 != 0;
  for (int64_t i = 0; i < len; ++i) {
    const int64_t tok = bos + i;
    // The next token's inputs are fetched while this one computes.
    const TokIn nxt = i + 1 < len ? load_in(tok + 1) : cur;
    prep_qk<K, VT>(sm, [&](int which, int) { return which == 0 ? cur.q : cur.k; },
                   p.l2norm, p.scale);
    if (tid < VT) sm.v[tid] = cur.v;
    const float decay = __expf(cur.g);
    const float beta = cur.b;
    T* o = reinterpret_cast<T*>(p.o) + (tok * p.HV + hv) * V + cs * VT;
    gdn_token<K, VT>(t, sm, decay, beta, [&](int c, float val) { o[c] = from_f32<T>(val); });
    if (per_token) {
      const int64_t sl = slot_of(i);
      if (sl >= 0 && sl < p.slots) store_tile<K, VT>(t, p.ht + sl * p.ht_slot_stride + col0, V);
    }
    cur = nxt;
  }
  if (!per_token) {
    if (p.inplace) {
      if (s0 >= 0 && s0 < p.slots && first_col >= 0)
        store_tile<K, VT>(t, p.ht + s0 * p.ht_slot_stride + col0, V);
    } else {
      store_tile<K, VT>(t, p.ht + n * p.ht_slot_stride + col0, V);
    }
  }
}

template <int K, int V, typename T, typename GT>
int rec_beta(const RecParams& p, xk_dtype bdt, hipStream_t s) {
  constexpr int NS = V == 128 ? 2 : 1;  // column slices per (sequence, head)
  const dim3 grid(p.N * p.HV * NS);
  switch (bdt) {
    case XK_F32: hipLaunchKernelGGL((gdn_recurrent_kernel<K, V, T, GT, float, NS>), grid, dim3(kThreads), 0, s, p); break;
    case XK_BF16: hipLaunchKernelGGL((gdn_recurrent_kernel<K, V, T, GT, bf16, NS>), grid, dim3(kThreads), 0, s, p); break;
    case XK_F16: hipLaunchKernelGGL((gdn_recurrent_kernel<K, V, T, GT, f16, NS>), grid, dim3(kThreads), 0, s, p); break;
    default: return XK_ERR_UNSUPPORTED;
  }
  return launch_status();
}

template <int K, int V, typename T>
int rec_g(const RecParams& p, xk_dtype gdt, xk_dtype bdt, hipStream_t s) {
  switch (gdt) {
    case XK_F32: return rec_beta<K, V, T, float>(p, bdt, s);
    case XK_BF16: return rec_beta<K, V, T, bf16>(p, bdt, s);
    case XK_F16: return rec_beta<K, V, T, f16>(p, bdt, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}

template <int K, int V>
int rec_t(const RecParams& p, xk_dtype dt, xk_dtype gdt, xk_dtype bdt, hipStream_t s) {
  switch (dt) {
    case XK_BF16: return rec_g<K, V, bf16>(p, gdt, bdt, s);
    case XK_F16: return rec_g<K, V, f16>(p, gdt, bdt, s);
    case XK_F32: return rec_g<K, V, float>(p, gdt, bdt, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}

// ---------------------------------------------------------------------------
// GDN gating, elementwise over [rows, heads], one element per lane (the
// most lanes in flight: every wave makes one load-compute-store pass, so the
// compute is on each wave's critical path and more elements per lane only
// lengthen it).  IT is the index type: 32-bit below 2^31 elements.
// ---------------------------------------------------------------------------
constexpr int kGateBlock = 128;  // 3.20 us at the bench shape, 3.23 with 256

template <typename AB, typename IT>
__global__ void __launch_bounds__(kGateBlock)
    gdn_gating_kernel(const float* __restrict__ A_log, const AB* __restrict__ a,
                      const AB* __restrict__ b, const float* __restrict__ dt_bias,
                      float* __restrict__ g, AB* __restrict__ beta_out, IT n, int heads,
                      float sp_beta, float inv_beta, float threshold) {
  const IT i = static_cast<IT>(blockIdx.x) * kGateBlock + static_cast<IT>(threadIdx.x);
  if (i >= n) return;
  const AB av = ld_stream(a + i);
  const AB bv = ld_stream(b + i);
  // A power-of-two head count (the common case) is a mask, not a division.
  const int h = (heads & (heads - 1)) == 0 ? static_cast<int>(i & static_cast<IT>(heads - 1))
                                           : static_cast<int>(i % static_cast<IT>(heads));
  st_stream(g + i, gdn_log_decay(to_f32(av) + dt_bias[h], A_log[h], sp_beta, inv_beta, threshold));
  st_stream(beta_out + i, sigmoid_to<AB>(to_f32(bv)));
}

// ---------------------------------------------------------------------------
// Decode step fused with the conv1d update.  One block per (batch row,
// qk-head): it owns the conv channels of that q head, that k head and the
// HV/H v heads of the group, so every conv channel and every state tile is
// read and written by exactly one block.
// ---------------------------------------------------------------------------
struct FusedParams {
  const void* x;  // mixed_qkv [B, D] (D = 2*H*K + HV*V)
  int64_t sx;
  void* conv_state;  // [lines, D, S]
  int64_t cs_line, cs_dim, cs_tok;
  int64_t conv_lines;
  int S;  // conv state_len
  const void* w;  // [D, W]
  int64_t w_dim, w_tap;
  const void* cbias;  // [D] or NULL
  xk_dtype wdt;
  const int32_t* conv_idx;
  int W;
  const void* g;  // [B, HV]
  const void* beta;
  float* state;  // [slots, HV, K, V]
  int64_t st_slot_stride;
  int64_t slots;
  const int32_t* ssm_idx;
  void* o;  // [B, HV, V]
  int64_t B;
  int H, HV;
  float scale;
  int l2norm;
  int32_t pad;
  // Conv state [lines, D, S] with S contiguous per channel and lines 16-byte
  // aligned, weights [D, W] contiguous in x's dtype, W - 1 == S <= 8: eight
  // channels per lane with 16-byte loads and stores.
  int conv_vec;
  // Gating mode: g holds a and beta holds b ([B, HV]); g = gdn_log_decay(a +
  // dt_bias, A_log) and beta = sigmoid(b), per head, in registers.
  int gating;
  const float* A_log;
  const float* dt_bias;
  float sp_beta, sp_thr;
};

// Conv update + SiLU of 8 consecutive channels c0..c0+7 of batch row b
// (FusedParams::conv_vec layout); writes the shifted state back.
template <typename T, int S>
__device__ __forceinline__ void conv8(const FusedParams& p, int64_t b, int64_t cslot,
                                      bool conv_ok, int64_t c0, float (&y)[8]) {
  using V8 = Vec<T, 8>;
  constexpr int W = S + 1;
  const V8 xv = ld_stream(reinterpret_cast<const V8*>(reinterpret_cast<const T*>(p.x) +
                                                      b * p.sx + c0));
  Arr<T, 8 * W> wv;  // weights of the 8 channels, channel-major
#pragma unroll
  for (int q = 0; q < W; ++q)
    *reinterpret_cast<V8*>(&wv.v[8 * q]) =
        reinterpret_cast<const V8*>(reinterpret_cast<const T*>(p.w) + c0 * W)[q];
  Arr<T, 8 * S> sv;  // state of the 8 channels, channel-major
  T* st = reinterpret_cast<T*>(p.conv_state) + cslot * p.cs_line + c0 * S;
  if (conv_ok) {
#pragma unroll
    for (int q = 0; q < S; ++q)
      *reinterpret_cast<V8*>(&sv.v[8 * q]) = ld_stream(reinterpret_cast<const V8*>(st) + q);
  } else {
#pragma unroll
    for (int e = 0; e < 8 * S; ++e) sv.v[e] = from_f32<T>(0.f);
  }
  Arr<T, 8 * S> ns;
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    float acc = p.cbias ? load_as_f32(p.cbias, c0 + c, p.wdt) : 0.f;
#pragma unroll
    for (int j = 0; j < S; ++j) acc = fmaf(to_f32(sv.v[c * S + j]), to_f32(wv.v[c * W + j]), acc);
    acc = fmaf(to_f32(xv.v[c]), to_f32(wv.v[c * W + S]), acc);
    y[c] = silu(acc);
#pragma unroll
    for (int j = 0; j + 1 < S; ++j) ns.v[c * S + j] = sv.v[c * S + j + 1];
    ns.v[c * S + S - 1] = xv.v[c];
  }
  if (conv_ok) {
#pragma unroll
    for (int q = 0; q < S; ++q)
      st_stream(reinterpret_cast<V8*>(st) + q, *reinterpret_cast<const V8*>(&ns.v[8 * q]));
  }
}

template <int K, int V, typename T, typename GT, typename BT>
__global__ void __launch_bounds__(kFusedThreads) gdn_conv_decode_kernel(FusedParams p) {
  constexpr int NT = kFusedThreads;
  __shared__ Smem<K, V, NT> sm;
  __shared__ float xv_lds[K * 2];          // q and k after conv + SiLU
  __shared__ float vv_lds[16][V];          // v heads of the group (R <= 16)
  const int64_t b = blockIdx.x / p.H;
  const int h = static_cast<int>(blockIdx.x % p.H);
  const int R = p.HV / p.H;
  const int tid = threadIdx.x;
  const int64_t cslot = p.conv_idx ? p.conv_idx[b] : b;
  const int64_t sslot = p.ssm_idx ? p.ssm_idx[b] : b;
  if (p.conv_idx && cslot == p.pad) return;  // padded batch row

  // Conv update for the group's channels: q (K), k (K), then R * V of v.
  const int nch = 2 * K + R * V;
  const bool conv_ok = cslot >= 0 && cslot < p.conv_lines;
  const bool st_ok = sslot >= 0 && sslot < p.slots;
  // The first v head's state tile is requested before the conv phase, so
  // its 64 KB stream overlaps the conv loads and arithmetic.
  Tile<K, V, NT> t;
  {
    float* sbase = p.state + sslot * p.st_slot_stride + static_cast<int64_t>(h) * R * K * V;
    if (st_ok) load_tile<K, V>(t, sbase); else zero_tile<K, V>(t);
  }
  // Global channel of group channel i: q (K), k (K), then R * V of v.
  auto chan = [&](int i) -> int64_t {
    if (i < K) return static_cast<int64_t>(h) * K + i;
    if (i < 2 * K) return static_cast<int64_t>(p.H) * K + static_cast<int64_t>(h) * K + (i - K);
    return 2 * static_cast<int64_t>(p.H) * K + static_cast<int64_t>(h) * R * V + (i - 2 * K);
  };
  auto put = [&](int i, float y) {
    if (i < 2 * K) xv_lds[i] = y;
    else vv_lds[(i - 2 * K) / V][(i - 2 * K) % V] = y;
  };
  if (p.conv_vec) {
    // 8 channels per lane (K and V are multiples of 8, so a group never
    // straddles the q / k / v parts).
    for (int i = tid * 8; i < nch; i += NT * 8) {
      float y[8];
      switch (p.S) {
        case 1: conv8<T, 1>(p, b, cslot, conv_ok, chan(i), y); break;
        case 2: conv8<T, 2>(p, b, cslot, conv_ok, chan(i), y); break;
        case 3: conv8<T, 3>(p, b, cslot, conv_ok, chan(i), y); break;
        default: conv8<T, 4>(p, b, cslot, conv_ok, chan(i), y); break;
      }
#pragma unroll
      for (int c = 0; c < 8; ++c) put(i + c, y[c]);
    }
  } else {
  for (int i = tid; i < nch; i += NT) {
    int64_t ch;
    if (i < K) ch = static_cast<int64_t>(h) * K + i;
    else if (i < 2 * K) ch = static_cast<int64_t>(p.H) * K + static_cast<int64_t>(h) * K + (i - K);
    else ch = 2 * static_cast<int64_t>(p.H) * K + static_cast<int64_t>(h) * R * V + (i - 2 * K);
    const float xc = ldf<T>(p.x, b * p.sx + ch);
    float acc = p.cbias ? load_as_f32(p.cbias, ch, p.wdt) : 0.f;
    T* st = reinterpret_cast<T*>(p.conv_state) + cslot * p.cs_line + ch * p.cs_dim;
    // window = cat(state[S-W+1 .. S-1], x)
    for (int j = 0; j < p.W - 1; ++j) {
      const float sv = conv_ok ? to_f32(st[(p.S - p.W + 1 + j) * p.cs_tok]) : 0.f;
      acc = fmaf(sv, load_as_f32(p.w, ch * p.w_dim + j * p.w_tap, p.wdt), acc);
    }
    acc = fmaf(xc, load_as_f32(p.w, ch * p.w_dim + (p.W - 1) * p.w_tap, p.wdt), acc);
    const float y = silu(acc);
    if (conv_ok) {  // shift the state left by one and append x
      for (int j = 0; j + 1 < p.S; ++j) st[j * p.cs_tok] = st[(j + 1) * p.cs_tok];
      st[(p.S - 1) * p.cs_tok] = reinterpret_cast<const T*>(p.x)[b * p.sx + ch];
    }
    put(i, y);
  }
  }
  __syncthreads();

  // Head j's tile is in `cur`; the next head's tile streams into `nxt`
  // while head j computes (two register tiles, unrolled by two): 204.4 ->
  // 197.8 us at config 5 on MI355X, the state stream no longer pausing
  // between the group's heads.
  Tile<K, V, NT> t2;
  auto head = [&](Tile<K, V, NT>& cur, Tile<K, V, NT>& nxt, int j) {
    const int hv = h * R + j;
    float* sbase = p.state + sslot * p.st_slot_stride + static_cast<int64_t>(hv) * K * V;
    if (j + 1 < R) {
      if (st_ok) load_tile<K, V>(nxt, sbase + K * V); else zero_tile<K, V>(nxt);
    }
    prep_qk<K, V>(sm, [&](int which, int e) { return xv_lds[which * K + e]; },
                  p.l2norm, p.scale);
    if (tid < V) sm.v[tid] = vv_lds[j][tid];
    float gv = ldf<GT>(p.g, b * p.HV + hv);
    float beta = p.beta ? ldf<BT>(p.beta, b * p.HV + hv) : 1.0f;
    if (p.gating) {
      gv = gdn_log_decay(gv + p.dt_bias[hv], p.A_log[hv], p.sp_beta, 1.0f / p.sp_beta, p.sp_thr);
      beta = sigmoid_exact(beta);
    }
    const float decay = __expf(gv);
    T* o = reinterpret_cast<T*>(p.o) + (b * p.HV + hv) * V;
    gdn_token<K, V>(cur, sm, decay, beta, [&](int c, float val) { o[c] = from_f32<T>(val); });
    if (st_ok) store_tile<K, V>(cur, sbase);
  };
  for (int j = 0; j < R; j += 2) {
    head(t, t2, j);
    if (j + 1 < R) head(t2, t, j + 1);
  }
}

template <int K, int V, typename T, typename GT>
int fused_beta(const FusedParams& p, xk_dtype bdt, hipStream_t s) {
  const dim3 grid(p.B * p.H);
  switch (bdt) {
    case XK_F32: hipLaunchKernelGGL((gdn_conv_decode_kernel<K, V, T, GT, float>), grid, dim3(kFusedThreads), 0, s, p); break;
    case XK_BF16: hipLaunchKernelGGL((gdn_conv_decode_kernel<K, V, T, GT, bf16>), grid, dim3(kFusedThreads), 0, s, p); break;
    case XK_F16: hipLaunchKernelGGL((gdn_conv_decode_kernel<K, V, T, GT, f16>), grid, dim3(kFusedThreads), 0, s, p); break;
    default: return XK_ERR_UNSUPPORTED;
  }
  return launch_status();
}

template <int K, int V, typename T>
int fused_g(const FusedParams& p, xk_dtype gdt, xk_dtype bdt, hipStream_t s) {
  switch (gdt) {
    case XK_F32: return fused_beta<K, V, T, float>(p, bdt, s);
    case XK_BF16: return fused_beta<K, V, T, bf16>(p, bdt, s);
    case XK_F16: return fused_beta<K, V, T, f16>(p, bdt, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}

}  // namespace
}  // namespace xk

using namespace xk;

extern "C" int xk_gdn_recurrent(
    const void* q, const void* k, const void* v, xk_dtype dtype, const void* g,
    xk_dtype g_dtype, const void* beta, xk_dtype beta_dtype, void* o,
    const float* initial_state, int64_t stride_h0_slot, float* final_state,
    int64_t stride_ht_slot, int64_t num_slots, const void* cu_seqlens,
    xk_dtype cu_dtype, const int32_t* ssm_state_indices, int64_t stride_idx_seq,
    int64_t stride_idx_tok, const int32_t* num_accepted_tokens, int64_t N,
    int64_t T, int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
    int use_qk_l2norm, int inplace_final_state, void* stream) {
  if (N < 0 || T < 0 || H <= 0 || HV <= 0 || HV % H != 0) return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(g_dtype) ||
      (beta && !is_float_dtype(beta_dtype)))
    return XK_ERR_UNSUPPORTED;
  if (cu_seqlens && cu_dtype != XK_I32 && cu_dtype != XK_I64) return XK_ERR_UNSUPPORTED;
  if (N == 0) return XK_OK;
  if (!q || !k || !v || !g || !o || !final_state) return XK_ERR_INVALID;
  if (inplace_final_state && !ssm_state_indices) return XK_ERR_INVALID;
  if (num_accepted_tokens && (!ssm_state_indices || !cu_seqlens || stride_idx_tok == 0))
    return XK_ERR_INVALID;
  if (!aligned(initial_state, 16) || !aligned(final_state, 16) ||
      stride_h0_slot % 4 || stride_ht_slot % 4)
    return XK_ERR_INVALID;
  RecParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = g;
  p.beta = beta;
  p.o = o;
  p.h0 = initial_state;
  p.ht = final_state;
  p.h0_slot_stride = stride_h0_slot;
  p.ht_slot_stride = stride_ht_slot;
  p.slots = num_slots;
  p.cu = cu_seqlens;
  p.cu_i64 = cu_dtype == XK_I64;
  p.idx = ssm_state_indices;
  p.idx_s0 = stride_idx_seq;
  p.idx_s1 = stride_idx_tok;
  p.accepted = num_accepted_tokens;
  p.N = N;
  p.T = T;
  p.H = static_cast<int>(H);
  p.HV = static_cast<int>(HV);
  p.scale = scale;
  p.l2norm = use_qk_l2norm;
  p.inplace = inplace_final_state;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const xk_dtype bdt = beta ? beta_dtype : XK_F32;
  if (K == 128 && V == 128) return rec_t<128, 128>(p, dtype, g_dtype, bdt, s);
  if (K == 64 && V == 64) return rec_t<64, 64>(p, dtype, g_dtype, bdt, s);
  if (K == 128 && V == 64) return rec_t<128, 64>(p, dtype, g_dtype, bdt, s);
  if (K == 64 && V == 128) return rec_t<64, 128>(p, dtype, g_dtype, bdt, s);
  return XK_ERR_UNSUPPORTED;
}

namespace {

// Shared argument checks and launch of the fused decode step; p.g / p.beta
// (and, with p.gating, a / b) are already set.
int conv_decode_launch(FusedParams& p, const void* mixed_qkv, int64_t stride_x_row,
                       void* conv_state, int64_t stride_cs_line, int64_t stride_cs_dim,
                       int64_t stride_cs_tok, int64_t conv_lines, int64_t conv_state_len,
                       const void* conv_weight, int64_t stride_w_dim, int64_t stride_w_tap,
                       const void* conv_bias, xk_dtype w_dtype, int64_t width,
                       const int32_t* conv_state_indices, int32_t pad_slot_id, xk_dtype g_dtype,
                       xk_dtype beta_dtype, float* ssm_state, int64_t stride_state_slot,
                       int64_t num_slots, const int32_t* ssm_state_indices, void* o, int64_t B,
                       int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
                       int use_qk_l2norm, xk_dtype dtype, void* stream) {
  if (B < 0 || H <= 0 || HV <= 0 || HV % H != 0 || HV / H > 16 || width < 1 ||
      conv_state_len < width - 1 || conv_state_len < 1)
    return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(g_dtype) || !is_float_dtype(w_dtype) ||
      (p.beta && !is_float_dtype(beta_dtype)))
    return XK_ERR_UNSUPPORTED;
  if (B == 0) return XK_OK;
  if (!mixed_qkv || !conv_state || !conv_weight || !p.g || !ssm_state || !o)
    return XK_ERR_INVALID;
  if (!aligned(ssm_state, 16) || stride_state_slot % 4) return XK_ERR_INVALID;
  if (K != 128 || V != 128) return XK_ERR_UNSUPPORTED;
  p.x = mixed_qkv;
  p.sx = stride_x_row;
  p.conv_state = conv_state;
  p.cs_line = stride_cs_line;
  p.cs_dim = stride_cs_dim;
  p.cs_tok = stride_cs_tok;
  p.conv_lines = conv_lines;
  p.S = static_cast<int>(conv_state_len);
  p.w = conv_weight;
  p.w_dim = stride_w_dim;
  p.w_tap = stride_w_tap;
  p.cbias = conv_bias;
  p.wdt = w_dtype;
  p.conv_idx = conv_state_indices;
  p.W = static_cast<int>(width);
  p.state = ssm_state;
  p.st_slot_stride = stride_state_slot;
  p.slots = num_slots;
  p.ssm_idx = ssm_state_indices;
  p.o = o;
  p.B = B;
  p.H = static_cast<int>(H);
  p.HV = static_cast<int>(HV);
  p.scale = scale;
  p.l2norm = use_qk_l2norm;
  p.pad = pad_slot_id;
  p.conv_vec = (dtype == XK_BF16 || dtype == XK_F16) && w_dtype == dtype &&
               stride_w_dim == width && stride_w_tap == 1 && stride_cs_tok == 1 &&
               stride_cs_dim == conv_state_len && conv_state_len == width - 1 &&
               conv_state_len <= 4 && stride_cs_line % 8 == 0 && stride_x_row % 8 == 0 &&
               aligned(mixed_qkv, 16) && aligned(conv_state, 16) && aligned(conv_weight, 16);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const xk_dtype bdt = p.beta ? beta_dtype : XK_F32;
  switch (dtype) {
    case XK_BF16: return fused_g<128, 128, bf16>(p, g_dtype, bdt, s);
    case XK_F16: return fused_g<128, 128, f16>(p, g_dtype, bdt, s);
    case XK_F32: return fused_g<128, 128, float>(p, g_dtype, bdt, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}

}  // namespace

extern "C" int xk_gdn_conv_decode(
    const void* mixed_qkv, int64_t stride_x_row, void* conv_state,
    int64_t stride_cs_line, int64_t stride_cs_dim, int64_t stride_cs_tok,
    int64_t conv_lines, int64_t conv_state_len, const void* conv_weight,
    int64_t stride_w_dim, int64_t stride_w_tap, const void* conv_bias,
    xk_dtype w_dtype, int64_t width, const int32_t* conv_state_indices,
    int32_t pad_slot_id, const void* g, xk_dtype g_dtype, const void* beta,
    xk_dtype beta_dtype, float* ssm_state, int64_t stride_state_slot,
    int64_t num_slots, const int32_t* ssm_state_indices, void* o, int64_t B,
    int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
    int use_qk_l2norm, xk_dtype dtype, void* stream) {
  FusedParams p{};
  p.g = g;
  p.beta = beta;
  return conv_decode_launch(p, mixed_qkv, stride_x_row, conv_state, stride_cs_line,
                            stride_cs_dim, stride_cs_tok, conv_lines, conv_state_len,
                            conv_weight, stride_w_dim, stride_w_tap, conv_bias, w_dtype, width,
                            conv_state_indices, pad_slot_id, g_dtype, beta_dtype, ssm_state,
                            stride_state_slot, num_slots, ssm_state_indices, o, B, H, HV, K, V,
                            scale, use_qk_l2norm, dtype, stream);
}

extern "C" int xk_gdn_conv_gating_decode(
    const void* mixed_qkv, int64_t stride_x_row, void* conv_state,
    int64_t stride_cs_line, int64_t stride_cs_dim, int64_t stride_cs_tok,
    int64_t conv_lines, int64_t conv_state_len, const void* conv_weight,
    int64_t stride_w_dim, int64_t stride_w_tap, const void* conv_bias,
    xk_dtype w_dtype, int64_t width, const int32_t* conv_state_indices,
    int32_t pad_slot_id, const float* A_log, const void* a, const float* dt_bias,
    const void* b, xk_dtype ab_dtype, float softplus_beta, float threshold,
    float* ssm_state, int64_t stride_state_slot, int64_t num_slots,
    const int32_t* ssm_state_indices, void* o, int64_t B, int64_t H, int64_t HV,
    int64_t K, int64_t V, float scale, int use_qk_l2norm, xk_dtype dtype,
    void* stream) {
  if (B > 0 && (!A_log || !dt_bias || !a || !b)) return XK_ERR_INVALID;
  if (softplus_beta == 0.f) return XK_ERR_INVALID;
  FusedParams p{};
  p.g = a;
  p.beta = b;
  p.gating = 1;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.sp_beta = softplus_beta;
  p.sp_thr = threshold;
  return conv_decode_launch(p, mixed_qkv, stride_x_row, conv_state, stride_cs_line,
                            stride_cs_dim, stride_cs_tok, conv_lines, conv_state_len,
                            conv_weight, stride_w_dim, stride_w_tap, conv_bias, w_dtype, width,
                            conv_state_indices, pad_slot_id, ab_dtype, ab_dtype, ssm_state,
                            stride_state_slot, num_slots, ssm_state_indices, o, B, H, HV, K, V,
                            scale, use_qk_l2norm, dtype, stream);
}

extern "C" int xk_fused_gdn_gating(const float* A_log, const void* a, const void* b,
                                   const float* dt_bias, float* g_out, void* beta_out,
                                   int64_t rows, int64_t heads, float softplus_beta,
                                   float threshold, xk_dtype ab_dtype, void* stream) {
  if (rows < 0 || heads <= 0 || heads > INT32_MAX || softplus_beta == 0.f) return XK_ERR_INVALID;
  if (!is_float_dtype(ab_dtype)) return XK_ERR_UNSUPPORTED;
  if (rows == 0) return XK_OK;
  if (!A_log || !a || !b || !dt_bias || !g_out || !beta_out) return XK_ERR_INVALID;
  const int64_t n = rows * heads;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hh = static_cast<int>(heads);
#define XK_GATE(T, IT)                                                                       \
  hipLaunchKernelGGL((gdn_gating_kernel<T, IT>), dim3(cdiv(n, kGateBlock)), dim3(kGateBlock), 0, \
                     s, A_log,                                                                 \
                     static_cast<const T*>(a), static_cast<const T*>(b), dt_bias, g_out,        \
                     static_cast<T*>(beta_out), static_cast<IT>(n), hh, softplus_beta,          \
                     1.0f / softplus_beta, threshold)
#define XK_GATE_T(T)                                   \
  if (n + kGateBlock < (int64_t{1} << 31)) {           \
    XK_GATE(T, uint32_t);                              \
  } else {                                             \
    XK_GATE(T, int64_t);                               \
  }
  switch (ab_dtype) {
    case XK_BF16: XK_GATE_T(bf16); break;
    case XK_F16: XK_GATE_T(f16); break;
    default: XK_GATE_T(float); break;
  }
#undef XK_GATE_T
#undef XK_GATE
  return launch_status();
}

extern "C" int xk_gdn_sigmoid_gating_update(
    const float* A_log, const void* a, const float* dt_bias, float softplus_beta,
    float threshold, const void* q, const void* k, const void* v, const void* b,
    xk_dtype ab_dtype, void* o, float* state, int64_t stride_state_slot,
    int64_t num_slots, const int32_t* state_indices, const int32_t* cu_seqlens,
    int64_t N, int64_t H, int64_t HV, int64_t K, int64_t V, float scale,
    int use_qk_l2norm, xk_dtype dtype, void* stream) {
  if (N < 0 || H <= 0 || HV <= 0 || HV % H != 0 || softplus_beta == 0.f) return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(ab_dtype)) return XK_ERR_UNSUPPORTED;
  if (N == 0) return XK_OK;
  if (!A_log || !a || !dt_bias || !q || !k || !v || !b || !o || !state || !state_indices ||
      !cu_seqlens)
    return XK_ERR_INVALID;
  if (!aligned(state, 16) || stride_state_slot % 4) return XK_ERR_INVALID;
  RecParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = a;
  p.beta = b;
  p.o = o;
  p.h0 = state;
  p.ht = state;
  p.h0_slot_stride = stride_state_slot;
  p.ht_slot_stride = stride_state_slot;
  p.slots = num_slots;
  p.cu = cu_seqlens;
  p.cu_i64 = 0;
  p.idx = state_indices;
  p.idx_s0 = 1;
  p.idx_s1 = 0;
  p.accepted = nullptr;
  p.N = N;
  p.T = 0;
  p.H = static_cast<int>(H);
  p.HV = static_cast<int>(HV);
  p.scale = scale;
  p.l2norm = use_qk_l2norm;
  p.inplace = 1;
  p.gating = 1;
  p.A_log = A_log;
  p.dt_bias = dt_bias;
  p.sp_beta = softplus_beta;
  p.sp_thr = threshold;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (K == 128 && V == 128) return rec_t<128, 128>(p, dtype, ab_dtype, ab_dtype, s);
  if (K == 64 && V == 64) return rec_t<64, 64>(p, dtype, ab_dtype, ab_dtype, s);
  if (K == 128 && V == 64) return rec_t<128, 64>(p, dtype, ab_dtype, ab_dtype, s);
  if (K == 64 && V == 128) return rec_t<64, 128>(p, dtype, ab_dtype, ab_dtype, s);
  return XK_ERR_UNSUPPORTED;
}
