// Fused split + per-head RMSNorm + neox RoPE for gfx950
// (xllm::kernel::npu::npu_split_rmsnorm_rope).
//
// Semantics follow the reference CPU golden
// (triton_npu/test/triton_split_rmsnorm_rope_test.cpp:88-136) and the
// Python reference (triton_npu/triton_src/test_split_rmsnorm_rope.py:
// 277-356): from a packed row [q_hidden | kv_hidden | kv_hidden]
//   q, k : per head of `head_dim`, n = x * 1/sqrt(mean(x^2) + eps) * w (+ b)
//          then out = n * cos + rotate_half(n) * sin,
//          rotate_half(n) = cat(-n[half:], n[:half])
//   v    : copied through.
// cos/sin are either per-token rows [T, head_dim] (the reference's
// interface) or computed in registers from integer positions and an fp32
// inverse-frequency table (neox layout: cos[d] = cos[d + half]).
//
// Design: one team of HALF/VEC lanes per (token, pair of heads) below 1024
// tokens, one wave per token from there.  Lane l holds the VEC-element
// slices [l*VEC, l*VEC+VEC) and [half + l*VEC, ...) of a head, so the
// rotate-half pairs (d, d + half) sit in the same lane and the rotation
// needs no data exchange.  A head's sum of squares is a shuffle reduction
// over the team; every global access is a 16-byte vector.
#include <type_traits>

#include "xk_common.h"

namespace xk {
namespace {

struct RopeParams {
  const void* qkv;
  int64_t stride_row;  // elements between tokens of qkv
  int64_t T;
  const void* sin;
  const void* cos;
  int64_t stride_sc;
  const void* pos;
  int pos_is_i64;
  const float* inv_freq;
  void* q;
  void* k;
  void* v;
  const void* qw;
  const void* qb;
  const void* kw;
  const void* kb;
  int hq, hkv;  // heads
  int64_t q_hidden, kv_hidden;
  float eps;
};

template <typename T, int N>
__device__ __forceinline__ void ld_f32(const T* p, float (&o)[N]) {
  const Vec<T, N> v = *reinterpret_cast<const Vec<T, N>*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = to_f32(v.v[i]);
}

template <typename T, int N>
__device__ __forceinline__ void vec_f32(const Vec<T, N>& v, float (&o)[N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) o[i] = to_f32(v.v[i]);
}

// Non-temporal store of N floats converted to T (outputs are written once).
template <typename T, int N>
__device__ __forceinline__ void st_f32(T* p, const float (&in)[N]) {
  Vec<T, N> v;
#pragma unroll
  for (int i = 0; i < N; ++i) v.v[i] = from_f32<T>(in[i]);
  st_stream(reinterpret_cast<Vec<T, N>*>(p), v);
}

// One team of HALF/VEC lanes per (token, group of G heads of one kind: all
// q, all k or all v; the host checks that G divides both head counts).  The
// team loads its cos/sin slice and weights once for its G heads.  Measured
// on MI355X at config 1 (256 tokens, fp32), against 5.0 us for one head per
// team: without the cos/sin and weight loads the kernel took 3.7 us (they
// were three times the x loads in vector-memory instructions); G = 2 takes
// 4.15 us, G = 4 4.5 us (half the waves, each twice as long); staging the
// block's cos/sin rows and weights in LDS instead (one small load per lane
// and a barrier) took 4.7-4.9 us.  Issuing the x loads first, before the
// q / k / v branch, was worth 0.5 us of the G = 2 gain.  The block size is
// chosen at launch (a whole number of waves, blockDim.x / kTeam teams).
template <typename T, typename A, int HD, int G>
__global__ void __launch_bounds__(1024) split_rmsnorm_rope_kernel(RopeParams p) {
  constexpr int kHalf = HD / 2;
  constexpr int kVec = (16 / sizeof(T)) < kHalf ? (16 / sizeof(T)) : kHalf;
  constexpr int kTeam = kHalf / kVec;
  static_assert(kTeam >= 1 && kTeam <= kWave && kWave % kTeam == 0, "team must fit a wave");
  const int teams = blockDim.x / kTeam;

  const int team = threadIdx.x / kTeam;
  const int lane = threadIdx.x % kTeam;
  const int groups = (p.hq + 2 * p.hkv) / G;
  const int64_t slot = static_cast<int64_t>(blockIdx.x) * teams + team;
  if (slot >= p.T * groups) return;  // whole team exits together
  const int64_t tok = slot / groups;
  const int h = static_cast<int>(slot - tok * groups) * G;  // first head of the group
  const int d0 = lane * kVec;

  const T* row = reinterpret_cast<const T*>(p.qkv) + tok * p.stride_row;
  using VT = Vec<T, kVec>;
  using VA = Vec<A, kVec>;
  const bool is_v = h >= p.hq + p.hkv;
  const bool is_q = h < p.hq;
  const int hh = is_v ? h - p.hq - p.hkv : (is_q ? h : h - p.hq);
  const T* src = row + (is_v ? p.q_hidden + p.kv_hidden : (is_q ? 0 : p.q_hidden)) +
                 static_cast<int64_t>(hh) * HD;
  VT xa[G], xb[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    xa[g] = ld_stream(reinterpret_cast<const VT*>(src + g * HD + d0));
    xb[g] = ld_stream(reinterpret_cast<const VT*>(src + g * HD + kHalf + d0));
  }
  if (is_v) {  // v: copy through
    T* dst = reinterpret_cast<T*>(p.v) + tok * p.kv_hidden + static_cast<int64_t>(hh) * HD;
#pragma unroll
    for (int g = 0; g < G; ++g) {
      st_stream(reinterpret_cast<VT*>(dst + g * HD + d0), xa[g]);
      st_stream(reinterpret_cast<VT*>(dst + g * HD + kHalf + d0), xb[g]);
    }
    return;
  }
  T* dst = reinterpret_cast<T*>(is_q ? p.q : p.k) +
           tok * (is_q ? p.q_hidden : p.kv_hidden) + static_cast<int64_t>(hh) * HD;
  const A* b = reinterpret_cast<const A*>(is_q ? p.qb : p.kb);

  // Every load of the group is issued before the first use, so the kernel
  // pays one memory latency: x (streamed), then weights, bias and sin/cos
  // (shared by many teams, served from cache).
  const A* w = reinterpret_cast<const A*>(is_q ? p.qw : p.kw);
  const VA wa = *reinterpret_cast<const VA*>(w + d0);
  const VA wb = *reinterpret_cast<const VA*>(w + kHalf + d0);
  // Without a bias (the usual case) no bias loads are issued: the branch is
  // uniform, and the two loads it saves per lane took config 1 from 5.24 to
  // 4.80 us on MI355X.
  float ba_f[kVec], bb_f[kVec];
  if (b) {
    ld_f32<A, kVec>(b + d0, ba_f);
    ld_f32<A, kVec>(b + kHalf + d0, bb_f);
  } else {
#pragma unroll
    for (int u = 0; u < kVec; ++u) ba_f[u] = bb_f[u] = 0.f;
  }
  VA ca, cb, sa, sb;
  if (!p.pos) {
    const A* cs = reinterpret_cast<const A*>(p.cos) + tok * p.stride_sc;
    const A* sn = reinterpret_cast<const A*>(p.sin) + tok * p.stride_sc;
    ca = *reinterpret_cast<const VA*>(cs + d0);
    cb = *reinterpret_cast<const VA*>(cs + kHalf + d0);
    sa = *reinterpret_cast<const VA*>(sn + d0);
    sb = *reinterpret_cast<const VA*>(sn + kHalf + d0);
  }

  float c1[kVec], c2[kVec], s1[kVec], s2[kVec];
  if (p.pos) {
    const float pos = p.pos_is_i64
                          ? static_cast<float>(reinterpret_cast<const int64_t*>(p.pos)[tok])
                          : static_cast<float>(reinterpret_cast<const int32_t*>(p.pos)[tok]);
    float f[kVec];
    ld_f32<float, kVec>(p.inv_freq + d0, f);
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      sincosf(pos * f[u], &s1[u], &c1[u]);
      s2[u] = s1[u];
      c2[u] = c1[u];
    }
  } else {
    vec_f32(ca, c1);
    vec_f32(cb, c2);
    vec_f32(sa, s1);
    vec_f32(sb, s2);
  }

#pragma unroll
  for (int g = 0; g < G; ++g) {
    float x1[kVec], x2[kVec];
    vec_f32(xa[g], x1);
    vec_f32(xb[g], x2);
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < kVec; ++u) ss = fmaf(x1[u], x1[u], fmaf(x2[u], x2[u], ss));
    ss = group_sum<kTeam>(ss);
    const float r = rsqrt_hw(ss * (1.0f / HD) + p.eps);
    float o1[kVec], o2[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const float n1 = fmaf(x1[u] * r, to_f32(wa.v[u]), ba_f[u]);
      const float n2 = fmaf(x2[u] * r, to_f32(wb.v[u]), bb_f[u]);
      o1[u] = n1 * c1[u] - n2 * s1[u];
      o2[u] = n2 * c2[u] + n1 * s2[u];
    }
    st_f32<T, kVec>(dst + g * HD + d0, o1);
    st_f32<T, kVec>(dst + g * HD + kHalf + d0, o2);
  }
}

// One wave per token.  The wave's 64 / kTeam teams take the token's heads
// in turn (team t: heads t, t + teams, ...) with the lane layout of
// split_rmsnorm_rope_kernel, so each lane forms its cos/sin (from the
// position, or loaded) and its q/k weights once and reuses them for every
// head of the token; computing sincosf per (token, head) made the
// positions mode VALU-bound at prefill sizes.
template <typename T, typename A, int HD, bool POS>
__global__ void __launch_bounds__(256) split_rmsnorm_rope_tok_kernel(RopeParams p) {
  constexpr int kHalf = HD / 2;
  constexpr int kVec = (16 / sizeof(T)) < kHalf ? (16 / sizeof(T)) : kHalf;
  constexpr int kTeam = kHalf / kVec;
  constexpr int kTpw = kWave / kTeam;  // teams per wave
  static_assert(kTeam >= 1 && kTeam <= kWave, "team must fit a wave");

  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (tok >= p.T) return;  // whole wave
  const int ln = threadIdx.x & 63;
  const int team = ln / kTeam;
  const int d0 = (ln % kTeam) * kVec;
  using VT = Vec<T, kVec>;
  using VA = Vec<A, kVec>;
  const T* row = reinterpret_cast<const T*>(p.qkv) + tok * p.stride_row;

  // cos / sin of the lane's dims d0.. and half + d0.. (equal in the
  // positions mode, where the neox rows repeat).
  constexpr int kCS = POS ? 1 : 2;
  float c[kCS][kVec], sn[kCS][kVec];
  if constexpr (POS) {
    // Every team of the wave needs the same kHalf values: each lane forms
    // cos / sin of dims ln, ln + 64, .. once (the same sincosf of the same
    // arguments) and the teams read theirs from the wave's LDS table.
    __shared__ __align__(16) float tab[4][2][kHalf];
    const int w = threadIdx.x >> 6;
    const float pos = p.pos_is_i64
                          ? static_cast<float>(reinterpret_cast<const int64_t*>(p.pos)[tok])
                          : static_cast<float>(reinterpret_cast<const int32_t*>(p.pos)[tok]);
#pragma unroll
    for (int i = ln; i < kHalf; i += kWave) sincosf(pos * p.inv_freq[i], &tab[w][1][i], &tab[w][0][i]);
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      c[0][u] = tab[w][0][d0 + u];
      sn[0][u] = tab[w][1][d0 + u];
    }
  } else {
    const A* cs = reinterpret_cast<const A*>(p.cos) + tok * p.stride_sc;
    const A* ss = reinterpret_cast<const A*>(p.sin) + tok * p.stride_sc;
    ld_f32<A, kVec>(cs + d0, c[0]);
    ld_f32<A, kVec>(cs + kHalf + d0, c[kCS - 1]);
    ld_f32<A, kVec>(ss + d0, sn[0]);
    ld_f32<A, kVec>(ss + kHalf + d0, sn[kCS - 1]);
  }
  // q and k weights (and biases; without one, the weight is read and
  // multiplied by zero), kept in their storage type until used.
  const A* qw = reinterpret_cast<const A*>(p.qw);
  const A* kw = reinterpret_cast<const A*>(p.kw);
  const A* qb = p.qb ? reinterpret_cast<const A*>(p.qb) : qw;
  const A* kb = p.kb ? reinterpret_cast<const A*>(p.kb) : kw;
  const float qbs = p.qb ? 1.f : 0.f, kbs = p.kb ? 1.f : 0.f;
  const VA wq1 = *reinterpret_cast<const VA*>(qw + d0);
  const VA wq2 = *reinterpret_cast<const VA*>(qw + kHalf + d0);
  const VA wk1 = *reinterpret_cast<const VA*>(kw + d0);
  const VA wk2 = *reinterpret_cast<const VA*>(kw + kHalf + d0);
  const VA bq1 = *reinterpret_cast<const VA*>(qb + d0);
  const VA bq2 = *reinterpret_cast<const VA*>(qb + kHalf + d0);
  const VA bk1 = *reinterpret_cast<const VA*>(kb + d0);
  const VA bk2 = *reinterpret_cast<const VA*>(kb + kHalf + d0);

  const int nqk = p.hq + p.hkv;
  auto src_of = [&](int h) {
    const bool is_q = h < p.hq;
    return row + (is_q ? 0 : p.q_hidden) + static_cast<int64_t>(is_q ? h : h - p.hq) * HD;
  };
  auto rope_head = [&](int h, const VT& xa, const VT& xb) {
    const bool is_q = h < p.hq;
    const int hh = is_q ? h : h - p.hq;
    T* dst = reinterpret_cast<T*>(is_q ? p.q : p.k) +
             tok * (is_q ? p.q_hidden : p.kv_hidden) + static_cast<int64_t>(hh) * HD;
    float x1[kVec], x2[kVec];
    vec_f32(xa, x1);
    vec_f32(xb, x2);
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < kVec; ++u) ss = fmaf(x1[u], x1[u], fmaf(x2[u], x2[u], ss));
    ss = group_sum<kTeam>(ss);
    const float r = rsqrt_hw(ss * (1.0f / HD) + p.eps);
    const float bs = is_q ? qbs : kbs;
    float o1[kVec], o2[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const float w1 = to_f32(is_q ? wq1.v[u] : wk1.v[u]);
      const float w2 = to_f32(is_q ? wq2.v[u] : wk2.v[u]);
      const float b1 = to_f32(is_q ? bq1.v[u] : bk1.v[u]) * bs;
      const float b2 = to_f32(is_q ? bq2.v[u] : bk2.v[u]) * bs;
      const float n1 = fmaf(x1[u] * r, w1, b1);
      const float n2 = fmaf(x2[u] * r, w2, b2);
      o1[u] = n1 * c[0][u] - n2 * sn[0][u];
      o2[u] = n2 * c[kCS - 1][u] + n1 * sn[kCS - 1][u];
    }
    st_f32<T, kVec>(dst + d0, o1);
    st_f32<T, kVec>(dst + kHalf + d0, o2);
  };
  for (int h = team; h < nqk; h += kTpw) {
    const T* sa = src_of(h);
    rope_head(h, ld_stream(reinterpret_cast<const VT*>(sa + d0)),
              ld_stream(reinterpret_cast<const VT*>(sa + kHalf + d0)));
  }
  for (int h = team; h < p.hkv; h += kTpw) {  // v: copy through
    const T* src = row + p.q_hidden + p.kv_hidden + static_cast<int64_t>(h) * HD;
    T* dst = reinterpret_cast<T*>(p.v) + tok * p.kv_hidden + static_cast<int64_t>(h) * HD;
    const VT a = ld_stream(reinterpret_cast<const VT*>(src + d0));
    const VT c = ld_stream(reinterpret_cast<const VT*>(src + kHalf + d0));
    st_stream(reinterpret_cast<VT*>(dst + d0), a);
    st_stream(reinterpret_cast<VT*>(dst + kHalf + d0), c);
  }
}

// Tokens from which the wave-per-token kernel is used: below it, a team per
// (token, head pair) gives the launch more waves to spread over the 256 CUs
// (at 256 tokens, one team per head took 5.3 us against 12.7 us).
constexpr int64_t kRopeTokKernelMin = 1024;

template <typename T, typename A, int HD>
int launch_rope(const RopeParams& p, hipStream_t s) {
  if (p.pos && p.T >= kRopeTokKernelMin) {
    hipLaunchKernelGGL((split_rmsnorm_rope_tok_kernel<T, A, HD, true>), dim3(cdiv(p.T, 4)),
                       dim3(256), 0, s, p);
    return launch_status();
  }
  if (p.T >= kRopeTokKernelMin) {
    hipLaunchKernelGGL((split_rmsnorm_rope_tok_kernel<T, A, HD, false>), dim3(cdiv(p.T, 4)),
                       dim3(256), 0, s, p);
    return launch_status();
  }
  constexpr int kHalf = HD / 2;
  constexpr int kVec = (16 / sizeof(T)) < kHalf ? (16 / sizeof(T)) : kHalf;
  constexpr int kTeam = kHalf / kVec;
  // Two heads per team when both head counts are even, else one.
  const int G = p.hq % 2 == 0 && p.hkv % 2 == 0 ? 2 : 1;
  const int64_t teams = p.T * ((p.hq + 2 * p.hkv) / G);
  if (teams == 0) return XK_OK;
  // As many blocks as CUs (or a multiple, when one CU's share of the teams
  // exceeds 1024 lanes), each the fewest whole waves that hold its share:
  // every CU gets the same work.  At config 1 (6144 teams of 16 lanes) that
  // is 256 blocks of 384 lanes: 3.99 us on MI355X, against 4.14 us for 384
  // blocks of 256 lanes (1.5 blocks per CU) and 4.2 us for 512 of 192.
  const int64_t cus = num_cus();
  int64_t nb = cus;
  while (cdiv(teams, nb) * kTeam > 1024) nb += cus;
  const int64_t lanes = cdiv(cdiv(teams, nb) * kTeam, kWave) * kWave;
  const dim3 grid(static_cast<unsigned>(cdiv(teams, lanes / kTeam)));
  if (G == 2)
    hipLaunchKernelGGL((split_rmsnorm_rope_kernel<T, A, HD, 2>), grid, dim3(lanes), 0, s, p);
  else
    hipLaunchKernelGGL((split_rmsnorm_rope_kernel<T, A, HD, 1>), grid, dim3(lanes), 0, s, p);
  return launch_status();
}

template <typename T, typename A>
int dispatch_hd(const RopeParams& p, int64_t hd, hipStream_t s) {
  switch (hd) {
    case 64: return launch_rope<T, A, 64>(p, s);
    case 128: return launch_rope<T, A, 128>(p, s);
    case 256: return launch_rope<T, A, 256>(p, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}

template <typename T>
int dispatch_aux(const RopeParams& p, int64_t hd, xk_dtype dt, xk_dtype aux,
                 hipStream_t s) {
  if (aux == dt) return dispatch_hd<T, T>(p, hd, s);
  if (aux == XK_F32) return dispatch_hd<T, float>(p, hd, s);
  return XK_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// In-place GPT-J (interleaved) RoPE on the last rope_dim elements of each row
// (xllm::kernel::npu::rope_inplace; reference rope_ref,
// triton_npu/triton_src/test_rope_inplace.py:66-94):
//   out[2i]   = x[2i]   cos[2i]   - x[2i+1] sin[2i]
//   out[2i+1] = x[2i+1] cos[2i+1] + x[2i]   sin[2i+1]
// with the sin/cos row of token row / head_num.  One lane per VEC elements
// (VEC/2 pairs), so each pair is lane-local; the untouched prefix of the row
// is never read.
// ---------------------------------------------------------------------------
template <typename T, typename A, int VEC>
__global__ void __launch_bounds__(256)
    rope_inplace_kernel(T* __restrict__ x, const A* __restrict__ sin, const A* __restrict__ cos,
                        int64_t rows, int head_num, int64_t sx, int64_t ssc, int64_t off,
                        int lanes_per_row) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t row = gid / lanes_per_row;
  if (row >= rows) return;
  const int e0 = static_cast<int>(gid - row * lanes_per_row) * VEC;
  T* xp = x + row * sx + off + e0;
  const int64_t tok = row / head_num;
  using VT = Vec<T, VEC>;
  using VA = Vec<A, VEC>;
  const VT xv = *reinterpret_cast<const VT*>(xp);
  const VA sv = *reinterpret_cast<const VA*>(sin + tok * ssc + e0);
  const VA cv = *reinterpret_cast<const VA*>(cos + tok * ssc + e0);
  VT ov;
#pragma unroll
  for (int u = 0; u < VEC; u += 2) {
    const float x0 = to_f32(xv.v[u]), x1 = to_f32(xv.v[u + 1]);
    ov.v[u] = from_f32<T>(x0 * to_f32(cv.v[u]) - x1 * to_f32(sv.v[u]));
    ov.v[u + 1] = from_f32<T>(x1 * to_f32(cv.v[u + 1]) + x0 * to_f32(sv.v[u + 1]));
  }
  *reinterpret_cast<VT*>(xp) = ov;
}

// One wave per token (vector path, rope_dim / VEC lanes per row dividing
// the wave): each lane loads its sin/cos vectors once and rotates the same
// slice of every head of the token, with a pass per 64 / lanes-per-row heads.
// NP > 0: the token has exactly NP passes, and every pass's row is loaded
// before the first store (NP rows in flight per lane; with a runtime pass
// count the loop runs load-store, load-store).  That took the bench shape
// (16 heads, 2 passes) from 17.4 to 17.1 us on MI355X.
template <typename T, typename A, int VEC, int LPR, int NP>
__global__ void __launch_bounds__(256)
    rope_inplace_tok_kernel(T* __restrict__ x, const A* __restrict__ sin,
                            const A* __restrict__ cos, int64_t tokens, int head_num, int64_t sx,
                            int64_t ssc, int64_t off) {
  constexpr int kRpp = kWave / LPR;  // rows (heads) per pass
  const int64_t tok = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (tok >= tokens) return;  // whole wave
  const int ln = threadIdx.x & 63;
  const int e0 = (ln % LPR) * VEC;
  using VT = Vec<T, VEC>;
  using VA = Vec<A, VEC>;
  auto rotate = [&](const VT& xv, const VA& sv, const VA& cv) {
    VT ov;
#pragma unroll
    for (int u = 0; u < VEC; u += 2) {
      const float x0 = to_f32(xv.v[u]), x1 = to_f32(xv.v[u + 1]);
      ov.v[u] = from_f32<T>(x0 * to_f32(cv.v[u]) - x1 * to_f32(sv.v[u]));
      ov.v[u + 1] = from_f32<T>(x1 * to_f32(cv.v[u + 1]) + x0 * to_f32(sv.v[u + 1]));
    }
    return ov;
  };
  if constexpr (NP > 0) {
    VT xv[NP];
    T* xp[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      xp[j] = x + (tok * head_num + ln / LPR + j * kRpp) * sx + off + e0;
      xv[j] = *reinterpret_cast<const VT*>(xp[j]);
    }
    const VA sv = *reinterpret_cast<const VA*>(sin + tok * ssc + e0);
    const VA cv = *reinterpret_cast<const VA*>(cos + tok * ssc + e0);
#pragma unroll
    for (int j = 0; j < NP; ++j) *reinterpret_cast<VT*>(xp[j]) = rotate(xv[j], sv, cv);
  } else {
    const VA sv = *reinterpret_cast<const VA*>(sin + tok * ssc + e0);
    const VA cv = *reinterpret_cast<const VA*>(cos + tok * ssc + e0);
    for (int h = ln / LPR; h < head_num; h += kRpp) {
      T* xp = x + (tok * head_num + h) * sx + off + e0;
      *reinterpret_cast<VT*>(xp) = rotate(*reinterpret_cast<const VT*>(xp), sv, cv);
    }
  }
}

template <typename T, typename A>
int launch_rope_inplace(void* x, const void* sin, const void* cos, int64_t rows, int head_num,
                        int64_t sx, int64_t ssc, int64_t hidden, int64_t rope_dim,
                        hipStream_t s) {
  constexpr int kV = 16 / sizeof(T) < 2 ? 2 : 16 / sizeof(T);
  const int64_t off = hidden - rope_dim;
  const bool vec = rope_dim % kV == 0 && off % kV == 0 && sx % kV == 0 && ssc % kV == 0 &&
                   aligned(x, 16) && aligned(sin, kV * sizeof(A)) &&
                   aligned(cos, kV * sizeof(A));
  const int v = vec ? kV : 2;
  const int lanes = static_cast<int>(rope_dim / v);
  const int64_t total = rows * lanes;
  const dim3 grid(cdiv(total, 256));
  T* xp = static_cast<T*>(x);
  const A* sp = static_cast<const A*>(sin);
  const A* cp = static_cast<const A*>(cos);
  // Whole tokens (rows = tokens x head_num) with 8 lanes per row.
  if (vec && lanes == 8 && rows % head_num == 0) {
    const int64_t tokens = rows / head_num;
    const dim3 tg(cdiv(tokens, 4));
#define XK_ROPE_TOK(NP) \
  hipLaunchKernelGGL((rope_inplace_tok_kernel<T, A, kV, 8, NP>), tg, dim3(256), 0, s, xp, sp, cp, \
                     tokens, head_num, sx, ssc, off)
    switch (head_num % 8 ? 0 : head_num / 8) {
      case 1: XK_ROPE_TOK(1); break;
      case 2: XK_ROPE_TOK(2); break;
      case 3: XK_ROPE_TOK(3); break;
      case 4: XK_ROPE_TOK(4); break;
      default: XK_ROPE_TOK(0); break;
    }
#undef XK_ROPE_TOK
    return launch_status();
  }
  if (vec)
    hipLaunchKernelGGL((rope_inplace_kernel<T, A, kV>), grid, dim3(256), 0, s, xp, sp, cp, rows,
                       head_num, sx, ssc, off, lanes);
  else
    hipLaunchKernelGGL((rope_inplace_kernel<T, A, 2>), grid, dim3(256), 0, s, xp, sp, cp, rows,
                       head_num, sx, ssc, off, lanes);
  return launch_status();
}

template <typename T>
int rope_inplace_aux(void* x, const void* sin, const void* cos, int64_t rows, int head_num,
                     int64_t sx, int64_t ssc, int64_t hidden, int64_t rope_dim, xk_dtype dt,
                     xk_dtype aux, hipStream_t s) {
  if (aux == dt)
    return launch_rope_inplace<T, T>(x, sin, cos, rows, head_num, sx, ssc, hidden, rope_dim, s);
  if (aux == XK_F32)
    return launch_rope_inplace<T, float>(x, sin, cos, rows, head_num, sx, ssc, hidden,
                                         rope_dim, s);
  return XK_ERR_UNSUPPORTED;
}

}  // namespace
}  // namespace xk

using namespace xk;

extern "C" int xk_rope_inplace(void* x, int64_t rows, int64_t head_num, int64_t stride_x_row,
                               int64_t hidden, const void* sin, const void* cos,
                               int64_t stride_sc_row, int64_t rope_dim, xk_dtype dtype,
                               xk_dtype sc_dtype, void* stream) {
  if (rows < 0 || head_num <= 0 || head_num > INT32_MAX || rope_dim <= 0 || rope_dim % 2 ||
      rope_dim > hidden || stride_x_row < hidden || stride_sc_row < rope_dim ||
      rope_dim / 2 > INT32_MAX)
    return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(sc_dtype)) return XK_ERR_UNSUPPORTED;
  if (rows == 0) return XK_OK;
  if (!x || !sin || !cos) return XK_ERR_INVALID;
  // Pairs are moved as aligned two-element vectors at the least.
  if ((hidden - rope_dim) % 2 || stride_x_row % 2 || stride_sc_row % 2 ||
      !aligned(x, 2 * elem_bytes(dtype)) || !aligned(sin, 2 * elem_bytes(sc_dtype)) ||
      !aligned(cos, 2 * elem_bytes(sc_dtype)))
    return XK_ERR_UNSUPPORTED;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int hn = static_cast<int>(head_num);
  switch (dtype) {
    case XK_F32:
      return rope_inplace_aux<float>(x, sin, cos, rows, hn, stride_x_row, stride_sc_row, hidden,
                                     rope_dim, dtype, sc_dtype, s);
    case XK_BF16:
      return rope_inplace_aux<bf16>(x, sin, cos, rows, hn, stride_x_row, stride_sc_row, hidden,
                                    rope_dim, dtype, sc_dtype, s);
    case XK_F16:
      return rope_inplace_aux<f16>(x, sin, cos, rows, hn, stride_x_row, stride_sc_row, hidden,
                                   rope_dim, dtype, sc_dtype, s);
    default:
      return XK_ERR_UNSUPPORTED;
  }
}

extern "C" int xk_split_rmsnorm_rope(
    const void* qkv, int64_t stride_qkv_row, int64_t num_tokens,
    const void* sin, const void* cos, int64_t stride_sc_row,
    const void* positions, xk_dtype pos_dtype, const float* inv_freq,
    void* q_out, void* k_out, void* v_out, const void* q_weight,
    const void* q_bias, const void* k_weight, const void* k_bias,
    xk_dtype aux_dtype, int64_t q_hidden, int64_t kv_hidden, int64_t head_dim,
    float eps, xk_dtype dtype, void* stream) {
  if (num_tokens < 0 || head_dim <= 0 || (head_dim & (head_dim - 1)) != 0 ||
      q_hidden <= 0 || kv_hidden <= 0 || q_hidden % head_dim != 0 ||
      kv_hidden % head_dim != 0 || stride_qkv_row < q_hidden + 2 * kv_hidden)
    return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(aux_dtype))
    return XK_ERR_UNSUPPORTED;
  if (positions && pos_dtype != XK_I32 && pos_dtype != XK_I64)
    return XK_ERR_UNSUPPORTED;
  if (num_tokens == 0) return XK_OK;
  if (!qkv || !q_out || !k_out || !v_out || !q_weight || !k_weight)
    return XK_ERR_INVALID;
  if (positions ? !inv_freq : (!sin || !cos || stride_sc_row < head_dim))
    return XK_ERR_INVALID;
  const int vec_bytes = 16;
  const int eb = elem_bytes(dtype);
  // Every row, head and half-head slice must start on a vector boundary.
  if ((stride_qkv_row * eb) % vec_bytes || !aligned(qkv, vec_bytes) ||
      !aligned(q_out, vec_bytes) || !aligned(k_out, vec_bytes) ||
      !aligned(v_out, vec_bytes))
    return XK_ERR_INVALID;
  // Aux vectors (weights, bias, sin/cos, inv_freq) are loaded with the
  // same element count as x: 16 bytes of x may mean 32 bytes of fp32 aux.
  const int aux_bytes = elem_bytes(aux_dtype) * (vec_bytes / eb);
  if (!aligned(q_weight, aux_bytes) || !aligned(k_weight, aux_bytes) ||
      (q_bias && !aligned(q_bias, aux_bytes)) ||
      (k_bias && !aligned(k_bias, aux_bytes)))
    return XK_ERR_INVALID;
  if (positions && !aligned(inv_freq, 4 * (vec_bytes / eb)))
    return XK_ERR_INVALID;
  if (!positions && ((stride_sc_row * elem_bytes(aux_dtype)) % aux_bytes ||
                     !aligned(sin, aux_bytes) || !aligned(cos, aux_bytes)))
    return XK_ERR_INVALID;
  RopeParams p{};
  p.qkv = qkv;
  p.stride_row = stride_qkv_row;
  p.T = num_tokens;
  p.sin = sin;
  p.cos = cos;
  p.stride_sc = stride_sc_row;
  p.pos = positions;
  p.pos_is_i64 = pos_dtype == XK_I64;
  p.inv_freq = inv_freq;
  p.q = q_out;
  p.k = k_out;
  p.v = v_out;
  p.qw = q_weight;
  p.qb = q_bias;
  p.kw = k_weight;
  p.kb = k_bias;
  p.hq = static_cast<int>(q_hidden / head_dim);
  p.hkv = static_cast<int>(kv_hidden / head_dim);
  p.q_hidden = q_hidden;
  p.kv_hidden = kv_hidden;
  p.eps = eps;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case XK_F32: return dispatch_aux<float>(p, head_dim, dtype, aux_dtype, s);
    case XK_BF16: return dispatch_aux<bf16>(p, head_dim, dtype, aux_dtype, s);
    case XK_F16: return dispatch_aux<f16>(p, head_dim, dtype, aux_dtype, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}
