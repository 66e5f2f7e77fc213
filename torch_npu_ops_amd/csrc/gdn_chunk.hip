// Chunked gated delta rule (prefill) for gfx950, chunk size 64.
//
// Semantics follow chunk_gated_delta_rule_full_op_ref
// (triton_npu/test/triton_chunk_gated_delta_rule_test.cpp:190-323), the
// pipeline of triton_npu/triton_src/chunk_gated_delta_rule/chunk.py:32-80.
// Per sequence, per v-head, per 64-token chunk with in-chunk cumulative
// log-decay gc (cumsum.py), beta b, keys k, queries q (scaled), values v and
// carried state S [K, V] (fp32):
//   M    = strict_tril(b_i (k_i . k_j) exp(gc_i - gc_j))     (kkt.py)
//   Ai   = (I + M)^-1                                        (solve_tril.py)
//   Vn   = Ai (b * (v - exp(gc) * (k S)))     == u - w S      (wy_fast.py,
//                                                            chunk_delta_h.py)
//   o    = exp(gc) * (q S) + tril(q k^T * exp(gc_i - gc_j)) Vn (chunk_o.py)
//   S   <- exp(gc_last) S + k^T (exp(gc_last - gc) * Vn)
// GQA: v-head hv uses qk-head hv / (HV / H).  Optional l2norm of q and k
// (npu_l2norm_last_dim, x / sqrt(sum x^2 + 1e-6)) is folded in as per-token
// row scales, so the matrix products always see the exact bf16 inputs.
//
// Three launches, no host synchronisation (capturable in a hipGraph):
//  * P0 (one small block) turns cu_seqlens into chunk offsets.
//  * P1, fully parallel, one wave per (chunk, v-head), computes everything
//    that does not depend on the carried state and writes one record per
//    (chunk, head) to the workspace:
//      - Ai = (I + M)^-1 as a bf16 hi/lo pair (hi + lo carries ~16 mantissa
//        bits).  K K^T runs on bf16 MFMA (exact products, fp32 sums); the
//        inverse inverts the two 32x32 diagonal blocks by forward
//        substitution (one lane per column) and forms the off-diagonal block
//        X10 = -X11 M10 X00 with hi/lo-split MFMAs;
//      - Aq = scale * tril(r_q r_k (q k^T) exp(gc_i - gc_j)) in bf16 (it only
//        feeds the bf16 output);
//      - per-token factors cq = scale exp(gc) r_q, ck = b exp(gc) r_k, b,
//        ed = r_k exp(gc_last - gc), and exp(gc_last).
//  * P2, sequential over the chunks of a sequence, one 512-lane block per
//    (sequence, v-head, 64-column V tile) (gdn_chunk_state8_kernel; a
//    256-lane block per 32-column tile when V is not a multiple of 64),
//    carries the fp32 state tile in registers through the short dependent
//    chain
//      KS = K S -> R = b v - ck KS -> Vn = Ai R -> S = e^gl S + K^T (ed Vn)
//    (hi/lo-split bf16 MFMAs keep the state within fp32-reference tolerance)
//    and emits o = cq (Q S) + Aq Vn.  Every global operand of chunk c+1 is
//    loaded while chunk c computes.  Blocks of one (sequence, head) share an
//    XCD (block id mod 8) and thus its L2 for the shared q/k/record reads.
#include <atomic>
#include <mutex>

#include "gdn_common.h"

namespace xk {
namespace {

using namespace gdn;

constexpr int kBVMax = 64;  // most V columns per P2 block (32 or 64)
constexpr int kTh = 256;  // threads per block
// Per-(chunk, head) record: ai_hi, ai_lo, aq, then the per-token factors
// (fp32 [5][64]: cq, ck, b, ed, exp(gc_last)).  Each matrix is stored as the
// MFMA A-operand images the state kernel loads, 1 KB each with lane l's 16
// bytes at byte 16 l: image (w, kk) holds rows 16 w + l % 16, columns
// 32 kk + 8 (l / 16) .. + 7, for wave w's rows.  The matrices are lower
// triangular, so the zero upper-right 32 x 32 block has no image: waves 0
// and 1 (rows 0..31) have only kk = 0, six images in all.  A lane-per-row
// layout (each load instruction touching 16 rows, 64 bytes of each) made
// the state kernel 15 us slower (262 -> 277 us at config 4 on MI355X): the
// loads of adjacent lanes were not contiguous.
constexpr int kMat = 6 * 512 * 2;  // bf16 bytes per matrix
constexpr int kRec = 3 * kMat + 5 * kC * 4;    // 19712 = 77 * 256
static_assert(kRec % 256 == 0, "records stay 256-byte aligned");

// Image of operand kk of wave w (waves 0, 1: kk = 0 only; their kk = 1
// maps to the kk = 0 image).
__device__ __forceinline__ int img_index(int w, int kk) { return w < 2 ? w : 2 * w - 2 + kk; }
// Padded rows of a sequence's last chunk store their (unused) outputs here,
// so that every store in the chunk loop is unconditional: gfx9 counts loads
// and stores in one in-order counter, and a store that only some paths
// issue makes the compiler wait for every outstanding prefetch.
constexpr int kDump = kC * kBVMax * 2;

struct ChunkParams {
  const void* q;  // [T, H, K]
  const void* k;
  const void* v;  // [T, HV, V]
  const void* g;  // [T, HV]
  const void* beta;
  void* o;  // [T, HV, V]
  const float* h0;  // [N, HV, K, V] or NULL
  float* ht;        // [N, HV, K, V] or NULL
  const void* cu;   // [N+1]
  int cu_i64;
  int32_t* chunk_off;  // [N+1] workspace
  int32_t* seq_order;  // [N] workspace: sequences, longest first
  int2* ctab;          // [NTmax] workspace: (first token, length) per chunk
  bf16* dump;          // [64 * kBVMax] workspace: sink for padded-row stores
  char* rec;           // [NTmax, HV] records of kRec bytes, workspace
  int64_t N, NTmax;
  int64_t T;  // token rows of q/k/v
  int H, HV;
  float scale;
  int l2norm;
};

__device__ __forceinline__ char* rec_at(const ChunkParams& p, int64_t c, int hv) {
  return p.rec + (c * p.HV + hv) * static_cast<int64_t>(kRec);
}

// Rows >= L of the K / Q operands (q4_load) repeat row L-1; here every
// consumer zeroes them through factors that are 0 there (beta, ck, ed, the
// masks of M and Aq).

// ---------------------------------------------------------------------------
// P1: one wave per (chunk, v-head); waves of a block are independent.
// ---------------------------------------------------------------------------

// r[row] = 1 / sqrt(sum x^2 + 1e-6) for the 64 rows of a chunk held as MFMA
// A operands (lane: row mi*16 + l15, elements kk*32 + 8*lg ...), or 1 when
// `on` is 0.  Sums use bf16 dot2 (exact products, fp32 accumulation).
template <int KK>
__device__ __forceinline__ void row_scales(const bf8_t (&x)[4][KK], float* r, int on) {
  const int lane = threadIdx.x & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  if (!on) {
    if (lg == 0)
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) r[mi * 16 + l15] = 1.0f;
    return;
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    float ss = 0.f;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const bf2_t pr = {x[mi][kk][e], x[mi][kk][e + 1]};
        ss = __builtin_amdgcn_fdot2_f32_bf16(pr, pr, ss, false);
      }
    ss += __shfl_xor(ss, 16, kWave);
    ss += __shfl_xor(ss, 32, kWave);
    if (lg == 0) r[mi * 16 + l15] = 1.0f / sqrtf(ss + 1e-6f);
  }
}

template <int K, typename GT, typename BT>
__global__ void __launch_bounds__(kTh) gdn_chunk_prep_kernel(ChunkParams p) {
  __shared__ __align__(16) float lds[4][kC][kLd];
  __shared__ float vec[4][4][kC];  // gc, beta, r_k, r_q per wave
  // Wave index in a scalar register: the exit below is then a scalar branch,
  // and the DPP transposes (q4_to_a) run with every lane of the wave active.
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  // Blocks take the head groups of one chunk before the next chunk, so
  // that the blocks in flight read whole token rows.
  const int hg4 = (p.HV + 3) >> 2;
  const int64_t c = blockIdx.x / hg4;
  const int hv = static_cast<int>(blockIdx.x % hg4) * 4 + wid;
  int64_t s;
  int L;
  if (p.N <= kWaveSeqs) {
    int64_t n;
    if (!wave_locate_chunk(p, c, n, s, L)) L = 0;
  } else {
    const int2 ce = p.ctab[c];  // (first token, length); length 0 past the last chunk
    s = ce.x;
    L = ce.y;
  }
  // Wave-uniform exit; the kernel has no block-level barriers.
  if (!(hv < p.HV && L > 0)) return;
  float (*X)[kLd] = lds[wid];
  float* gcv = vec[wid][0];
  float* btv = vec[wid][1];
  float* rkv = vec[wid][2];
  float* rqv = vec[wid][3];
  const int hq = hv / (p.HV / p.H);
  constexpr int KK = K / 32;
  const int64_t rs = static_cast<int64_t>(p.H) * K;

  // K rows of the chunk as MFMA operands (A and B^T read the same rows),
  // loaded quad-contiguously (q4_load; rows >= L repeat row L-1).  Every
  // product here pairs two such operands, so q4_to_a's key order needs no
  // change on the other side.
  static_assert(K == 128, "q4 operand loads are 16 x 128");
  const bf16* kbase = reinterpret_cast<const bf16*>(p.k) + static_cast<int64_t>(hq) * K;
  const bf16* qbase = reinterpret_cast<const bf16*>(p.q) + static_cast<int64_t>(hq) * K;
  bf8_t kop[4][KK];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
    q4_load([&](int r) { return kbase + (s + min(mi * 16 + r, L - 1)) * rs; }, kop[mi]);
  // Per-token g (inclusive scan within the chunk) and beta; padded rows 0
  // (loads clamped to row L-1, then selected away).
  const int lt = min(lane, L - 1);
  const float graw = ldf<GT>(p.g, (s + lt) * p.HV + hv);
  const float braw = ldf<BT>(p.beta, (s + lt) * p.HV + hv);
  float gv = lane < L ? graw : 0.f;
  const float bv = lane < L ? braw : 0.f;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const float t = __shfl_up(gv, o, kWave);
    if (lane >= o) gv += t;
  }
  gcv[lane] = gv;
  btv[lane] = bv;
  // Row scales r = 1 / sqrt(sum x^2 + 1e-6) of the rows this lane holds
  // (row mi*16 + l15; the four lg lanes hold its four 32-wide pieces), or 1
  // without the in-op l2norm.
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) q4_to_a(kop[mi]);
  row_scales<KK>(kop, rkv, p.l2norm);
  __builtin_amdgcn_wave_barrier();

  // M = strict_tril(b_i r_i r_j (k_i . k_j) exp(gc_i - gc_j)) into X (the
  // ten lower 16x16 tiles; the strictly upper ones are never read).  The
  // product K_nj K_mi^T is tile (mi, nj) transposed, so a lane holds row
  // mi*16 + l15, columns nj*16 + 4 lg .. + 3, written as one 16-byte vector.
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int row = mi * 16 + l15;
    const float fr = btv[row] * rkv[row], gr = gcv[row];
#pragma unroll
    for (int nj = 0; nj <= mi; ++nj) {
      f4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) a = mfma16(kop[nj][kk], kop[mi][kk], a);
      f4_t m;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = nj * 16 + 4 * lg + i;
        m[i] = row > col ? fr * rkv[col] * a[i] * __expf(gr - gcv[col]) : 0.f;
      }
      *reinterpret_cast<f4_t*>(&X[row][nj * 16 + 4 * lg]) = m;
    }
  }
  __builtin_amdgcn_wave_barrier();

  // Q rows, loaded before the inverse so that their latency hides behind
  // it (252 VGPRs with them live; the LDS footprint already limits the
  // kernel to two waves per SIMD, so the registers cost no occupancy).
  // Measured on MI355X at config 4: 87.6 -> 84.4 us.
  bf8_t qop[4][KK];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
    q4_load([&](int r) { return qbase + (s + min(mi * 16 + r, L - 1)) * rs; }, qop[mi]);

  invert_unit_lower(X);  // X = (I + M)^-1, row-major

  char* rec = rec_at(p, c, hv);
  __bf16* aih = reinterpret_cast<__bf16*>(rec);
  __bf16* ail = reinterpret_cast<__bf16*>(rec + kMat);
  __bf16* aqp = reinterpret_cast<__bf16*>(rec + 2 * kMat);
  float* sc = reinterpret_cast<float*>(rec + 3 * kMat);
  // Ai as hi and lo bf16 operand images.  Store j writes image j, one
  // contiguous KB, so every store instruction writes whole cache lines;
  // image j = img_index(w, kk) for (w, kk) = (0,0) (1,0) (2,0) (2,1) (3,0)
  // (3,1).  Lane l reads X row 16 w + l % 16 from column 32 kk + 8 (l / 16):
  // 8 lanes of one b128 read cover all 32 banks (row stride 68 = 4 mod 32).
  auto tri_row = [&](int j) { return 16 * (j < 2 ? j : 2 + ((j - 2) >> 1)) + l15; };
  auto tri_col = [&](int j) { return 32 * (j < 2 ? 0 : (j - 2) & 1) + 8 * lg; };
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    bf8_t h, l;
    split8(&X[tri_row(j)][tri_col(j)], h, l);
    *reinterpret_cast<bf8_t*>(aih + 512 * j + 8 * lane) = h;
    *reinterpret_cast<bf8_t*>(ail + 512 * j + 8 * lane) = l;
  }
  __builtin_amdgcn_wave_barrier();

#pragma unroll
  for (int mi = 0; mi < 4; ++mi) q4_to_a(qop[mi]);
  row_scales<KK>(qop, rqv, p.l2norm);
  __builtin_amdgcn_wave_barrier();

  // Aq = scale * tril(r_q r_k (q k^T) exp(gc_i - gc_j)), rows < L, formed
  // transposed like M (K_nj Q_mi^T) for 16-byte row writes.
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int row = mi * 16 + l15;
    const float fr = p.scale * rqv[row], gr = gcv[row];
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      f4_t a = {0.f, 0.f, 0.f, 0.f};
      if (nj <= mi) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) a = mfma16(kop[nj][kk], qop[mi][kk], a);
      }
      f4_t val;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = nj * 16 + 4 * lg + i;
        val[i] = nj <= mi && row >= col && row < L ? fr * rkv[col] * a[i] * __expf(gr - gcv[col])
                                                    : 0.f;
      }
      *reinterpret_cast<f4_t*>(&X[row][nj * 16 + 4 * lg]) = val;
    }
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < 6; ++j) {
    bf8_t h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = static_cast<__bf16>(X[tri_row(j)][tri_col(j) + e]);
    *reinterpret_cast<bf8_t*>(aqp + 512 * j + 8 * lane) = h;
  }

  // Per-token factors (lane = token); rows >= L are zero.
  const float gl = __shfl(gv, L - 1, kWave);
  const bool in = lane < L;
  const float eg = __expf(gv);
  sc[0 * kC + lane] = in ? p.scale * eg * rqv[lane] : 0.f;
  sc[1 * kC + lane] = in ? bv * eg * rkv[lane] : 0.f;
  sc[2 * kC + lane] = bv;
  sc[3 * kC + lane] = in ? rkv[lane] * __expf(gl - gv) : 0.f;
  sc[4 * kC + lane] = __expf(gl);
}

// ---------------------------------------------------------------------------
// P2: sequential chunk loop per (sequence, v-head, 32-column V tile), for V
// not a multiple of 64 (the 64-column kernel below covers the rest).
// ---------------------------------------------------------------------------
constexpr int kLt = kC + 8;  // bf16 LDS row stride (144 B: 16-byte aligned)

// The fp32 state tile itself lives in registers (each wave owns K/4 of its
// rows, in MFMA C layout); LDS holds its bf16 hi / lo copy, the B operand of
// K S, refreshed once per chunk.
template <int K, int BV>
struct __align__(16) P2Smem {
  __bf16 sb[2][BV][K + 8];    // state hi / lo, transposed: sb[h][v][k]
  __bf16 kr[2][kC * K];       // chunk key rows (kr_off layout), double-buffered
  __bf16 rt[2][BV][kLt];      // R transposed, hi / lo
  __bf16 vt[BV][kLt];         // Vn transposed (bf16, for the output)
  __bf16 dt[2][BV][kLt];      // (ed * Vn) transposed, hi / lo
};

// Operands one lane reads from global memory for one chunk, in three
// groups.  Those the chunk consumes first are double-buffered (loaded a whole
// chunk ahead).  The two later groups have one buffer each, refilled with
// the next chunk's operands right after their last use in the current chunk
// (so each load has most of a chunk to land) -- this keeps two waves per
// SIMD.
template <int KK, int NV32>
struct EarlyOps {
  bf8_t kA[KK];          // K rows wid*16.. as q4_load leaves them (stored as they are
                         // into the chunk's key tile, store_kr_q4)
  bf8_t vA[NV32];        // v row wid*16 + l15, tile columns 32j + 8*lg .. + 7
                         // (A layout; select_op turns it into C layout)
  f4_t ck, bt;           // factors of rows wid*16 + 4*lg + i
  float egl;             // exp(gc_last)
};
struct InvOps {          // consumed by Vn = Ai R and ed * Vn
  bf8_t aiH[2], aiL[2];  // Ai rows wid*16 + l15, hi / lo
  f4_t ed;
};
template <int KK>
struct OutOps {          // consumed by the output o = cq (Q S) + Aq Vn
  bf8_t qA[KK];          // Q rows wid*16.., as kA
  bf8_t aq[2];           // Aq rows wid*16 + l15
  float cq;              // factor of row wid*16 + l15
};

// Token row of q/k/v for C-layout row `r` (rows >= L read row L-1: finite,
// and zeroed by their factors).
template <int K, int BV>
__device__ __forceinline__ void load_early(const ChunkParams& p, EarlyOps<K / 32, BV / 32>& ops,
                                           int64_t s, int L, int64_t cidx, int hv, int hq,
                                           uint32_t vrow, int vcol0) {
  const int lane = threadIdx.x & 63, wid = wave_index();
  const int l15 = lane & 15, lg = lane >> 4;
  const uint32_t rs = static_cast<uint32_t>(p.H) * K;
  const WaveRows wr = wave_rows(s, L, wid);
  const char* kb = reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.k) +
                                                 wr.row0 * rs + hq * K);
  q4_load_b(kb, 2 * rs, wr.lw, ops.kA);
  const char* vb = reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.v) +
                                                 wr.row0 * vrow + vcol0);
#pragma unroll
  for (int j = 0; j < BV / 32; ++j)
    ops.vA[j] = *reinterpret_cast<const bf8_t*>(vb + row_off(l15, wr.lw, 2 * vrow, 32 * j + 8 * lg));
  const float* sc = reinterpret_cast<const float*>(rec_at(p, cidx, hv) + 3 * kMat);
  const int r4 = wid * 16 + 4 * lg;
  ops.ck = *reinterpret_cast<const f4_t*>(sc + 1 * kC + r4);
  ops.bt = *reinterpret_cast<const f4_t*>(sc + 2 * kC + r4);
  ops.egl = sc[4 * kC];
}

__device__ __forceinline__ void load_inv(const ChunkParams& p, InvOps& ops, int64_t cidx,
                                         int hv) {
  const int lane = threadIdx.x & 63, wid = wave_index();
  const int lg = lane >> 4;
  const char* rec = rec_at(p, cidx, hv);
  const float* sc = reinterpret_cast<const float*>(rec + 3 * kMat);
  // Rows 0..31 have no stored columns 32..63 (zero): their kk = 1 operand
  // re-reads the kk = 0 image, keeping every load unconditional, and is
  // never multiplied (the Vn product skips it).
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const char* img = rec + img_index(wid, kk) * 1024;
    ops.aiH[kk] = *reinterpret_cast<const bf8_t*>(img + 16 * lane);
    ops.aiL[kk] = *reinterpret_cast<const bf8_t*>(img + kMat + 16 * lane);
  }
  ops.ed = *reinterpret_cast<const f4_t*>(sc + 3 * kC + wid * 16 + 4 * lg);
}

template <int K>
__device__ __forceinline__ void load_out(const ChunkParams& p, OutOps<K / 32>& ops, int64_t s,
                                         int L, int64_t cidx, int hv, int hq) {
  const int lane = threadIdx.x & 63, wid = wave_index();
  const int l15 = lane & 15;
  const uint32_t rs = static_cast<uint32_t>(p.H) * K;
  const WaveRows wr = wave_rows(s, L, wid);
  const char* qb = reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.q) +
                                                 wr.row0 * rs + hq * K);
  q4_load_b(qb, 2 * rs, wr.lw, ops.qA);
  const char* rec = rec_at(p, cidx, hv);
  const float* sc = reinterpret_cast<const float*>(rec + 3 * kMat);
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)  // waves 0, 1: kk = 1 as for Ai
    ops.aq[kk] = *reinterpret_cast<const bf8_t*>(rec + 2 * kMat + img_index(wid, kk) * 1024 + 16 * lane);
  ops.cq = sc[0 * kC + wid * 16 + l15];
}

template <int K, typename T, int BV>
__global__ void __launch_bounds__(kTh) __attribute__((amdgpu_waves_per_eu(BV == 32 ? 2 : 1)))
gdn_chunk_state_kernel(ChunkParams p, int nvt) {
  static_assert(BV == 32 || BV == 64, "V tile of 32 or 64 columns");
  __shared__ P2Smem<K, BV> sm;
  constexpr int KK = K / 32;
  constexpr int NJ = BV / 16;  // 16-column tiles per block
  const int tid = threadIdx.x;
  const int wid = wave_index();
  const int lane = tid & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  // XCD-aware mapping: the nvt V tiles of one (sequence, head) get block ids
  // that are equal modulo 8, i.e. run on the same XCD and share its L2.
  // Items are dispatched longest sequence first, so the longest chains start
  // in the first wave of resident blocks.
  const int64_t w = blockIdx.x;
  const int64_t xcd = w & 7, r = w >> 3;
  const int vt = static_cast<int>(r % nvt);
  const int64_t item = (r / nvt) * 8 + xcd;  // (sequence rank, head) index
  if (item >= p.N * p.HV) return;            // whole block
  int64_t n, cidx0;
  find_ranked_seq(p, item / p.HV, n, cidx0);
  const int hv = state_head(static_cast<int>(item % p.HV), p.HV, p.H);
  const int hq = hv / (p.HV / p.H);
  const int V = nvt * BV;
  const int v0 = vt * BV;
  const int64_t bos = cu_at(p, n), eos = cu_at(p, n + 1);
  // Chunks of this sequence; the NTmax bound keeps a malformed cu_seqlens
  // (never a well-formed one) from reading past the workspace.
  const int64_t nch = max<int64_t>(0, min<int64_t>((eos - bos + kC - 1) / kC, p.NTmax - cidx0));

  // State rows (k) wid*(K/4) + m2*16 + 4*lg + i, columns nj*16 + l15.
  constexpr int M2 = K / 64;
  f4_t sreg[M2][NJ];
#pragma unroll
  for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kr = wid * (K / 4) + m2 * 16 + 4 * lg + i;
        sreg[m2][nj][i] = p.h0 ? p.h0[((n * p.HV + hv) * K + kr) * V + v0 + nj * 16 + l15] : 0.f;
      }
  // bf16 hi / lo copy of the state for the K S operand.
  auto publish_state = [&]() {
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        Vec<__bf16, 4> h, l;
        split4(sreg[m2][nj], h, l);
        const int k0 = wid * (K / 4) + m2 * 16 + 4 * lg;
        *reinterpret_cast<Vec<__bf16, 4>*>(&sm.sb[0][nj * 16 + l15][k0]) = h;
        *reinterpret_cast<Vec<__bf16, 4>*>(&sm.sb[1][nj * 16 + l15][k0]) = l;
      }
  };
  publish_state();
  const uint32_t vrow = static_cast<uint32_t>(p.HV) * V;  // v / o token stride
  const int vcol0 = hv * V + v0;
  const bf8_t sel[2] = {select_op(0), select_op(1)};
  EarlyOps<KK, BV / 32> opsA, opsB;
  InvOps inv;
  OutOps<KK> outo;
  if (nch > 0) {
    const int L0 = static_cast<int>(min<int64_t>(kC, eos - bos));
    load_early<K, BV>(p, opsA, bos, L0, cidx0, hv, hq, vrow, vcol0);
    // Keep the early group ahead of the others, in loop order: the loop's
    // wait counts are fixed by the shortest distance (in memory operations)
    // between a load and its first use over every path, this one included,
    // and an early load scheduled last here would make every chunk wait for
    // the previous chunk's most recent loads.
    __builtin_amdgcn_sched_barrier(0);
    load_inv(p, inv, cidx0, hv);
    __builtin_amdgcn_sched_barrier(0);
    load_out<K>(p, outo, bos, L0, cidx0, hv, hq);
    store_kr_q4(sm.kr[0], opsA.kA, wid);
  }
  __syncthreads();

  // One chunk: `cur` holds its early operands, `nxt` receives the next
  // chunk's; `inv` and `outo` are refilled with the next chunk's operands
  // right after their last use here.  The last chunk "prefetches" itself
  // again (unused), so that every memory operation of the loop is
  // unconditional.
  auto step = [&](const EarlyOps<KK, BV / 32>& cur, EarlyOps<KK, BV / 32>& nxt, int64_t ci) {
    const int64_t s = bos + ci * kC;
    const int L = static_cast<int>(min<int64_t>(kC, eos - s));
    const int64_t cn = min(ci + 1, nch - 1);
    const int64_t sn = bos + cn * kC;
    const int Ln = static_cast<int>(min<int64_t>(kC, eos - sn));
    load_early<K, BV>(p, nxt, sn, Ln, cidx0 + cn, hv, hq, vrow, vcol0);

    // KS = K S (hi/lo S): rows wid*16.., columns nj*16..; K's rows come
    // from the chunk's key tile.
    const __bf16* kr = sm.kr[ci & 1];
    f4_t ks[NJ];
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) ks[nj] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const bf8_t ka = kr_a(kr, wid, kk);
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        const bf8_t sh = *reinterpret_cast<const bf8_t*>(&sm.sb[0][nj * 16 + l15][kk * 32 + 8 * lg]);
        const bf8_t sl = *reinterpret_cast<const bf8_t*>(&sm.sb[1][nj * 16 + l15][kk * 32 + 8 * lg]);
        ks[nj] = mfma16(ka, sh, ks[nj]);
        ks[nj] = mfma16(ka, sl, ks[nj]);
      }
    }
    // R = b v - ck KS  ->  rt (transposed, hi / lo); padded rows are 0.
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) {
      Vec<__bf16, 4> h, l;
      const f4_t vc = mfma16(cur.vA[nj >> 1], sel[nj & 1], f4_t{0.f, 0.f, 0.f, 0.f});
      f4_t rv;
#pragma unroll
      for (int i = 0; i < 4; ++i) rv[i] = cur.bt[i] * vc[i] - cur.ck[i] * ks[nj][i];
      split4(rv, h, l);
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.rt[0][nj * 16 + l15][wid * 16 + 4 * lg]) = h;
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.rt[1][nj * 16 + l15][wid * 16 + 4 * lg]) = l;
    }
    __syncthreads();  // (1) rt complete

    // Vn = Ai R.
    f4_t vn[NJ];
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) {
      vn[nj] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        if (kk * 32 > wid * 16 + 15) continue;  // zero block of Ai (not stored)
        const bf8_t rh = *reinterpret_cast<const bf8_t*>(&sm.rt[0][nj * 16 + l15][kk * 32 + 8 * lg]);
        const bf8_t rl = *reinterpret_cast<const bf8_t*>(&sm.rt[1][nj * 16 + l15][kk * 32 + 8 * lg]);
        vn[nj] = mfma_split3(inv.aiH[kk], inv.aiL[kk], rh, rl, vn[nj]);
      }
    }
    // Vn -> vt (bf16), ed * Vn -> dt (hi / lo).
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) {
      Vec<__bf16, 4> b, h, l;
      f4_t d;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        b.v[i] = static_cast<__bf16>(vn[nj][i]);
        d[i] = inv.ed[i] * vn[nj][i];
      }
      split4(d, h, l);
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.vt[nj * 16 + l15][wid * 16 + 4 * lg]) = b;
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.dt[0][nj * 16 + l15][wid * 16 + 4 * lg]) = h;
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.dt[1][nj * 16 + l15][wid * 16 + 4 * lg]) = l;
    }
    load_inv(p, inv, cidx0 + cn, hv);  // this chunk is done with `inv`
    // (Q S)^T = S^T Q^T with the hi part of S: the output is produced
    // transposed (lane: token wid*16 + l15, columns 4*lg .. 4*lg + 3), so
    // each lane stores one 8-byte vector per column tile.  The S^T A operand
    // is the same sb read as S's B operand, and Q^T's B operand is Q's A
    // operand.  It must read sb before barrier 2: after it, a wave that is
    // ahead may already publish the next state into sb.
    q4_to_a(outo.qA);
    f4_t qs[NJ];
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) {
      qs[nj] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const bf8_t sh = *reinterpret_cast<const bf8_t*>(&sm.sb[0][nj * 16 + l15][q4_key(kk, lg)]);
        qs[nj] = mfma16(sh, outo.qA[kk], qs[nj]);
      }
    }
    __syncthreads();  // (2) vt, dt complete; rt and sb reads done

    // o^T = cq (Q S)^T + Vn^T Aq^T (Vn^T's A operand is the vt read that
    // was Vn's B operand; Aq^T's B operand is Aq's A operand).
    // The MFMA leaves lane (g = lane / 16, t = lane % 16) with row t,
    // columns nj*16 + 4 g ..; before the store, lane (r = lane / 16, a =
    // lane / 4 % 4, b = lane % 4) pulls (ds_bpermute) the values of row
    // 4 a + r, column group b from lane 16 b + 4 a + r.  Each quad then
    // writes 32 contiguous bytes of one row, where the MFMA layout had the 4
    // lanes of a quad write 4 different rows (7 us of the state kernel at
    // config 4 on MI355X).
    static_assert(sizeof(T) == 2, "two dwords per 4-column group");
    {
      const int row = wid * 16 + quad_row(), qb = quad_col();
      T* orow = row < L ? reinterpret_cast<T*>(p.o) + static_cast<uint64_t>(s + row) * vrow + vcol0
                        : reinterpret_cast<T*>(p.dump) + row * BV;
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        f4_t acc;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = outo.cq * qs[nj][i];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          if (kk * 32 > wid * 16 + 15) continue;  // Aq columns beyond the diagonal
          const bf8_t vb = *reinterpret_cast<const bf8_t*>(&sm.vt[nj * 16 + l15][kk * 32 + 8 * lg]);
          acc = mfma16(vb, outo.aq[kk], acc);
        }
        Vec<T, 4> ov;
#pragma unroll
        for (int i = 0; i < 4; ++i) ov.v[i] = from_f32<T>(acc[i]);
        *reinterpret_cast<u32x2*>(orow + nj * 16 + 4 * qb) = quad_rows(__builtin_bit_cast(u32x2, ov));
      }
    }
    load_out<K>(p, outo, sn, Ln, cidx0 + cn, hv, hq);  // this chunk is done with `outo`

    // S <- exp(gc_last) S + K^T (ed Vn) on the wave's register rows, then
    // its bf16 copy (every wave finished reading sb before barrier 2).
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2) {
      const int mi = wid * M2 + m2;
      bf8_t ka[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) ka[kk] = kr_at(kr, mi, kk);
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        f4_t acc = sreg[m2][nj];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= cur.egl;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf8_t dh = *reinterpret_cast<const bf8_t*>(&sm.dt[0][nj * 16 + l15][kk * 32 + 8 * lg]);
          const bf8_t dl = *reinterpret_cast<const bf8_t*>(&sm.dt[1][nj * 16 + l15][kk * 32 + 8 * lg]);
          acc = mfma16(ka[kk], dh, acc);
          acc = mfma16(ka[kk], dl, acc);
        }
        sreg[m2][nj] = acc;
      }
    }
    publish_state();
    store_kr_q4(sm.kr[(ci + 1) & 1], nxt.kA, wid);
    __syncthreads();  // (3) state copy, next keys complete; vt / dt / key reads done
  };
  // Unrolled by two so the operand buffers swap roles without copies.
  for (int64_t ci = 0; ci < nch; ci += 2) {
    step(opsA, opsB, ci);
    if (ci + 1 < nch) step(opsB, opsA, ci + 1);
  }
  if (p.ht) {
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kr = wid * (K / 4) + m2 * 16 + 4 * lg + i;
          p.ht[((n * p.HV + hv) * K + kr) * V + v0 + nj * 16 + l15] = sreg[m2][nj][i];
        }
  }
}

// ---------------------------------------------------------------------------
// P2 with one 512-lane block per (sequence, v-head, 64-column V tile): eight
// waves, wave (wr = wid % 4, cg = wid / 4) owning token rows 16 wr .., state
// key rows 32 wr .. and columns 32 cg .. of the tile, exactly the share of a
// wave of gdn_chunk_state_kernel.  The two column groups share the chunk's
// key and query rows: each wave loads 8 of the 64 rows of each as whole
// rows, into a key tile (read as rows for K S and transposed for the state
// update) and a query tile (read as rows for Q S, so Q needs no register
// transpose).  One block per CU (132 KB of LDS), two waves per SIMD as with
// two 256-lane blocks; the loop issues 31% fewer VALU instructions than the
// 256-lane kernel's.  Measured on MI355X at config 4: 226.8 -> 221.6 us.
// The per-token factors (cq, ck, beta, ed) reach the waves through a 1 KB
// LDS tile that every wave fills with one load of the record's factor
// block, instead of four loads of its own rows of them; e^{g_last} is a
// scalar load.  That is 4 fewer vector-memory instructions per wave and
// step and 24 fewer VGPRs (222 -> 198): 223.9 -> 221.5 us.
// ---------------------------------------------------------------------------
constexpr int kTh8 = 512;

// The transposed tiles below (sb8_off, t8_off) are unpadded and swizzled.

template <int K>
struct __align__(16) P2Smem8 {
  __bf16 sb[2][64 * K];     // state hi / lo, transposed: [v][k] (sb8_off)
  __bf16 kr[2][kC * K];     // chunk key rows (kr_off layout), double-buffered
  __bf16 qr[kC * K];        // chunk query rows (kr_off layout)
  __bf16 rt[2][64 * kC];    // R transposed, hi / lo (t8_off)
  __bf16 vt[64 * kC];       // Vn transposed (bf16, for the output)
  __bf16 dt[2][64 * kC];    // (ed * Vn) transposed, hi / lo
  float fac[2][4 * kC];     // per-token factors cq, ck, beta, ed of the chunk, double-buffered
};

struct EarlyOps8 {
  bf8_t kraw[2], qraw[2];  // key / query rows 16 wr + 8 cg + 4 j + lane / 16, chunk lane % 16
  bf8_t vA;                // v row 16 wr + l15, columns 32 cg + 8 lg .. + 7 (A layout)
  f4_t fac;                // factor floats 4 lane .. 4 lane + 3 of the record
  float egl;
};
struct InvOps8 {
  bf8_t aiH[2], aiL[2];
};
struct OutOps8 {
  bf8_t aq[2];
};
typedef __attribute__((address_space(4))) const float cfloat_t;

template <int K>
__global__ void __launch_bounds__(kTh8) __attribute__((amdgpu_waves_per_eu(2)))
gdn_chunk_state8_kernel(ChunkParams p, int nvt) {
  constexpr int BV = 64;
  static_assert(K == 128, "key rows of 128");
  __shared__ P2Smem8<K> sm;
  constexpr int KK = K / 32;
  constexpr int NJ = 2;  // 16-column tiles per wave
  const int tid = threadIdx.x;
  const int wid = wave_index();
  // Waves w and w + 4 share a SIMD; they take token rows wr and 3 - wr, so
  // that every SIMD gets the same share of the triangular products (Ai and
  // Aq hold 1, 1, 2, 2 nonzero 32-wide pieces for rows 0..3).  Measured on
  // MI355X at config 4: 283.0 -> 280.1 us per call.
  const int cg = wid >> 2, wr = cg ? 3 - (wid & 3) : (wid & 3), cb = 32 * cg;
  const int lane = tid & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  const int rl = lane >> 4, ch = lane & 15;  // whole-row loads: row in a load, 16-byte chunk
  const int64_t w = blockIdx.x;
  const int64_t xcd = w & 7, r = w >> 3;
  const int vt = static_cast<int>(r % nvt);
  const int64_t item = (r / nvt) * 8 + xcd;
  if (item >= p.N * p.HV) return;
  int64_t n, cidx0;
  find_ranked_seq(p, item / p.HV, n, cidx0);
  const int hv = state_head(static_cast<int>(item % p.HV), p.HV, p.H);
  const int hq = hv / (p.HV / p.H);
  const int V = nvt * BV;
  const int v0 = vt * BV;
  const int64_t bos = cu_at(p, n), eos = cu_at(p, n + 1);
  const int64_t nch = max<int64_t>(0, min<int64_t>((eos - bos + kC - 1) / kC, p.NTmax - cidx0));

  constexpr int M2 = K / 64;
  f4_t sreg[M2][NJ];
#pragma unroll
  for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kr = wr * (K / 4) + m2 * 16 + 4 * lg + i;
        sreg[m2][nj][i] =
            p.h0 ? p.h0[((n * p.HV + hv) * K + kr) * V + v0 + cb + nj * 16 + l15] : 0.f;
      }
  auto publish_state = [&]() {
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        Vec<__bf16, 4> h, l;
        split4(sreg[m2][nj], h, l);
        const int k0 = wr * (K / 4) + m2 * 16 + 4 * lg;
        *reinterpret_cast<Vec<__bf16, 4>*>(&sm.sb[0][sb8_off(cb + nj * 16 + l15, k0)]) = h;
        *reinterpret_cast<Vec<__bf16, 4>*>(&sm.sb[1][sb8_off(cb + nj * 16 + l15, k0)]) = l;
      }
  };
  publish_state();
  const uint32_t vrow = static_cast<uint32_t>(p.HV) * V;
  const int vcol0 = hv * V + v0 + cb;
  const uint32_t rb = static_cast<uint32_t>(p.H) * K * 2;  // q / k row bytes
  const bf8_t sel[2] = {select_op(0), select_op(1)};

  auto load_early8 = [&](EarlyOps8& o, int64_t s, int L, int64_t cidx) {
    const char* kb = reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.k) + s * p.H * K + hq * K);
    const char* qb = reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.q) + s * p.H * K + hq * K);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t off = static_cast<uint32_t>(min(wr * 16 + cg * 8 + 4 * j + rl, L - 1)) * rb + 16u * ch;
      o.kraw[j] = *reinterpret_cast<const bf8_t*>(kb + off);
      o.qraw[j] = *reinterpret_cast<const bf8_t*>(qb + off);
    }
    const WaveRows wrs = wave_rows(s, L, wr);
    const char* vb = reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.v) +
                                                   wrs.row0 * vrow + vcol0);
    o.vA = *reinterpret_cast<const bf8_t*>(vb + row_off(l15, wrs.lw, 2 * vrow, 8 * lg));
    // The factor block (cq, ck, beta, ed: 1 KB) in one load per wave; the
    // wave-uniform e^{g_last} through the scalar cache.
    const char* sc = rec_at(p, cidx, hv) + 3 * kMat;
    o.fac = *reinterpret_cast<const f4_t*>(sc + 16 * lane);
    o.egl = *(cfloat_t*)(sc + 16 * kC);
  };
  auto load_inv8 = [&](InvOps8& o, int64_t cidx) {
    const char* rec = rec_at(p, cidx, hv);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const char* img = rec + img_index(wr, kk) * 1024;
      o.aiH[kk] = *reinterpret_cast<const bf8_t*>(img + 16 * lane);
      o.aiL[kk] = *reinterpret_cast<const bf8_t*>(img + kMat + 16 * lane);
    }
  };
  auto load_out8 = [&](OutOps8& o, int64_t cidx) {
    const char* rec = rec_at(p, cidx, hv);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      o.aq[kk] = *reinterpret_cast<const bf8_t*>(rec + 2 * kMat + img_index(wr, kk) * 1024 + 16 * lane);
  };
  // Every wave writes the same factor bytes (one 16-byte store per lane).
  auto store_fac = [&](float* f, const f4_t& v) { *reinterpret_cast<f4_t*>(f + 4 * lane) = v; };
  auto store_rows = [&](__bf16* tile, const bf8_t (&raw)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<bf8_t*>(tile + kr_off(wr * 16 + cg * 8 + 4 * j + rl, ch)) = raw[j];
  };

  EarlyOps8 opsA, opsB;
  InvOps8 inv;
  OutOps8 outo;
  if (nch > 0) {
    const int L0 = static_cast<int>(min<int64_t>(kC, eos - bos));
    load_early8(opsA, bos, L0, cidx0);
    __builtin_amdgcn_sched_barrier(0);
    load_inv8(inv, cidx0);
    __builtin_amdgcn_sched_barrier(0);
    load_out8(outo, cidx0);
    store_rows(sm.kr[0], opsA.kraw);
    store_rows(sm.qr, opsA.qraw);
    store_fac(sm.fac[0], opsA.fac);
  }
  __syncthreads();

  auto step = [&](const EarlyOps8& cur, EarlyOps8& nxt, int64_t ci) {
    const int64_t s = bos + ci * kC;
    const int L = static_cast<int>(min<int64_t>(kC, eos - s));
    const int64_t cn = min(ci + 1, nch - 1);
    const int64_t sn = bos + cn * kC;
    const int Ln = static_cast<int>(min<int64_t>(kC, eos - sn));
    load_early8(nxt, sn, Ln, cidx0 + cn);

    const __bf16* kr = sm.kr[ci & 1];
    const float* fc = sm.fac[ci & 1];
    const f4_t ck = *reinterpret_cast<const f4_t*>(fc + 1 * kC + wr * 16 + 4 * lg);
    const f4_t bt = *reinterpret_cast<const f4_t*>(fc + 2 * kC + wr * 16 + 4 * lg);
    f4_t ks[NJ];
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) ks[nj] = f4_t{0.f, 0.f, 0.f, 0.f};
    // The scheduler's small-GEMM interleaving of LDS reads and MFMAs for the
    // K S and state-update products: 221.6 -> 216.6 us at config 4 on MI355X
    // (the variant for wider tiles, iglp_opt(1), took 237 us).
    __builtin_amdgcn_iglp_opt(0);
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const bf8_t ka = kr_a(kr, wr, kk);
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        const bf8_t sh = *reinterpret_cast<const bf8_t*>(&sm.sb[0][sb8_off(cb + nj * 16 + l15, kk * 32 + 8 * lg)]);
        const bf8_t sl = *reinterpret_cast<const bf8_t*>(&sm.sb[1][sb8_off(cb + nj * 16 + l15, kk * 32 + 8 * lg)]);
        ks[nj] = mfma16(ka, sh, ks[nj]);
        ks[nj] = mfma16(ka, sl, ks[nj]);
      }
    }
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) {
      Vec<__bf16, 4> h, l;
      const f4_t vc = mfma16(cur.vA, sel[nj], f4_t{0.f, 0.f, 0.f, 0.f});
      f4_t rv;
#pragma unroll
      for (int i = 0; i < 4; ++i) rv[i] = bt[i] * vc[i] - ck[i] * ks[nj][i];
      split4(rv, h, l);
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.rt[0][t8_off(cb + nj * 16 + l15, wr * 16 + 4 * lg)]) = h;
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.rt[1][t8_off(cb + nj * 16 + l15, wr * 16 + 4 * lg)]) = l;
    }
    __syncthreads();  // (1)

    const f4_t ed = *reinterpret_cast<const f4_t*>(fc + 3 * kC + wr * 16 + 4 * lg);
    f4_t vn[NJ];
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) {
      vn[nj] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        if (kk * 32 > wr * 16 + 15) continue;
        const bf8_t rh = *reinterpret_cast<const bf8_t*>(&sm.rt[0][t8_off(cb + nj * 16 + l15, kk * 32 + 8 * lg)]);
        const bf8_t rl2 = *reinterpret_cast<const bf8_t*>(&sm.rt[1][t8_off(cb + nj * 16 + l15, kk * 32 + 8 * lg)]);
        vn[nj] = mfma_split3(inv.aiH[kk], inv.aiL[kk], rh, rl2, vn[nj]);
      }
    }
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) {
      Vec<__bf16, 4> b, h, l;
      f4_t d;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        b.v[i] = static_cast<__bf16>(vn[nj][i]);
        d[i] = ed[i] * vn[nj][i];
      }
      split4(d, h, l);
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.vt[t8_off(cb + nj * 16 + l15, wr * 16 + 4 * lg)]) = b;
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.dt[0][t8_off(cb + nj * 16 + l15, wr * 16 + 4 * lg)]) = h;
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.dt[1][t8_off(cb + nj * 16 + l15, wr * 16 + 4 * lg)]) = l;
    }
    load_inv8(inv, cidx0 + cn);
    // (Q S)^T = S^T Q^T: Q's rows from the query tile, keys in natural order.
    f4_t qs[NJ];
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj) qs[nj] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const bf8_t qa = kr_a(sm.qr, wr, kk);
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        const bf8_t sh = *reinterpret_cast<const bf8_t*>(&sm.sb[0][sb8_off(cb + nj * 16 + l15, kk * 32 + 8 * lg)]);
        qs[nj] = mfma16(sh, qa, qs[nj]);
      }
    }
    __syncthreads();  // (2) vt, dt complete; rt, sb and query reads done

    {
      const int row = wr * 16 + quad_row(), qb = quad_col();
      const float cq = fc[0 * kC + wr * 16 + l15];
      bf16* orow = row < L ? reinterpret_cast<bf16*>(p.o) + static_cast<uint64_t>(s + row) * vrow + vcol0
                           : reinterpret_cast<bf16*>(p.dump) + row * BV + cb;
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        f4_t acc;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = cq * qs[nj][i];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          if (kk * 32 > wr * 16 + 15) continue;
          const bf8_t vb = *reinterpret_cast<const bf8_t*>(&sm.vt[t8_off(cb + nj * 16 + l15, kk * 32 + 8 * lg)]);
          acc = mfma16(vb, outo.aq[kk], acc);
        }
        Vec<bf16, 4> ov;
#pragma unroll
        for (int i = 0; i < 4; ++i) ov.v[i] = from_f32<bf16>(acc[i]);
        *reinterpret_cast<u32x2*>(orow + nj * 16 + 4 * qb) = quad_rows(__builtin_bit_cast(u32x2, ov));
      }
    }
    load_out8(outo, cidx0 + cn);

    __builtin_amdgcn_iglp_opt(0);
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2) {
      const int mi = wr * M2 + m2;
      bf8_t ka[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) ka[kk] = kr_at(kr, mi, kk);
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        f4_t acc = sreg[m2][nj];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= cur.egl;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf8_t dh = *reinterpret_cast<const bf8_t*>(&sm.dt[0][t8_off(cb + nj * 16 + l15, kk * 32 + 8 * lg)]);
          const bf8_t dl = *reinterpret_cast<const bf8_t*>(&sm.dt[1][t8_off(cb + nj * 16 + l15, kk * 32 + 8 * lg)]);
          acc = mfma16(ka[kk], dh, acc);
          acc = mfma16(ka[kk], dl, acc);
        }
        sreg[m2][nj] = acc;
      }
    }
    publish_state();
    store_rows(sm.kr[(ci + 1) & 1], nxt.kraw);
    store_rows(sm.qr, nxt.qraw);
    store_fac(sm.fac[(ci + 1) & 1], nxt.fac);
    __syncthreads();  // (3)
  };
  for (int64_t ci = 0; ci < nch; ci += 2) {
    step(opsA, opsB, ci);
    if (ci + 1 < nch) step(opsB, opsA, ci + 1);
  }
  if (p.ht) {
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kr = wr * (K / 4) + m2 * 16 + 4 * lg + i;
          p.ht[((n * p.HV + hv) * K + kr) * V + v0 + cb + nj * 16 + l15] = sreg[m2][nj][i];
        }
  }
}

template <int K, typename GT, typename BT>
int launch_chunk(const ChunkParams& p, int64_t V, hipStream_t s) {
  int st;
  if (p.N > kWaveSeqs) {  // else the kernels look chunks up themselves
    hipLaunchKernelGGL(chunk_offsets_kernel<ChunkParams>, dim3(1), dim3(256), 0, s, p,
                       p.seq_order, p.ctab, p.NTmax);
    if ((st = launch_status())) return st;
  }
  const int64_t prep_blocks = p.NTmax * ((p.HV + 3) / 4);
  if (prep_blocks > INT32_MAX) return XK_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((gdn_chunk_prep_kernel<K, GT, BT>), dim3(static_cast<uint32_t>(prep_blocks)),
                     dim3(kTh), 0, s, p);
  st = launch_status();
  if (st) return st;
  const int64_t items = p.N * p.HV;
  if (V % 64 == 0) {
    const int nvt = static_cast<int>(V / 64);
    const int64_t blocks = cdiv(items, 8) * 8 * nvt;
    hipLaunchKernelGGL((gdn_chunk_state8_kernel<K>), dim3(blocks), dim3(kTh8), 0, s, p, nvt);
  } else {
    constexpr int BV = 32;
    const int nvt = static_cast<int>(V / BV);
    const int64_t blocks = cdiv(items, 8) * 8 * nvt;
    hipLaunchKernelGGL((gdn_chunk_state_kernel<K, bf16, BV>), dim3(blocks), dim3(kTh), 0, s, p, nvt);
  }
  return launch_status();
}

// g and beta each come in fp32 or bf16 (chunk.py's callers pass fp32 g and
// bf16 beta).
template <int K, typename GT>
int chunk_beta(const ChunkParams& p, int64_t V, xk_dtype bdt, hipStream_t s) {
  if (bdt == XK_F32) return launch_chunk<K, GT, float>(p, V, s);
  if (bdt == XK_BF16) return launch_chunk<K, GT, bf16>(p, V, s);
  return XK_ERR_UNSUPPORTED;
}

int64_t nt_max(int64_t total_tokens, int64_t N) { return total_tokens / kC + N; }

}  // namespace
}  // namespace xk

using namespace xk;

extern "C" int64_t xk_gdn_chunk_workspace_bytes(int64_t total_tokens, int64_t num_seqs,
                                                int64_t HV) {
  if (total_tokens < 0 || num_seqs < 0 || HV <= 0) return -1;
  const int64_t nt = nt_max(total_tokens, num_seqs);
  return align256(4 * (num_seqs + 1)) + align256(4 * num_seqs) + align256(8 * nt) + kDump +
         nt * HV * kRec;
}

namespace xk {
namespace {

// Argument checks shared by xk_gdn_chunk_fwd and xk_gdn_chunk_fwd_noalloc
// (everything but the workspace).  *empty is set for a call with no work
// (N or total_tokens 0), which returns XK_OK before its pointers are
// checked.
int chunk_args_status(const void* q, const void* k, const void* v, xk_dtype dtype,
                      const void* g, xk_dtype g_dtype, const void* beta, xk_dtype beta_dtype,
                      const void* o, const void* cu_seqlens, xk_dtype cu_dtype, int64_t N,
                      int64_t total_tokens, int64_t H, int64_t HV, int64_t K, int64_t V,
                      bool* empty) {
  *empty = false;
  if (N < 0 || total_tokens < 0 || H <= 0 || HV <= 0 || HV % H != 0)
    return XK_ERR_INVALID;
  // bf16 only, as the reference entry point (q/k feed the bf16 MFMA as-is).
  if (dtype != XK_BF16) return XK_ERR_UNSUPPORTED;
  if (g_dtype != XK_F32 && g_dtype != XK_BF16) return XK_ERR_UNSUPPORTED;
  if (beta_dtype != XK_F32 && beta_dtype != XK_BF16) return XK_ERR_UNSUPPORTED;
  if (cu_dtype != XK_I32 && cu_dtype != XK_I64) return XK_ERR_UNSUPPORTED;
  if (K != 128 || V % 32 != 0 || V <= 0) return XK_ERR_UNSUPPORTED;
  // Row pitches of q / k and v / o in bytes feed 24-bit multiplies.
  if (H * K * 2 >= (int64_t{1} << 24) || HV * V * 2 >= (int64_t{1} << 24))
    return XK_ERR_UNSUPPORTED;
  if (N == 0 || total_tokens == 0) {
    *empty = true;
    return XK_OK;
  }
  // Token indices travel as int32 in the chunk table.
  if (total_tokens > INT32_MAX - kC) return XK_ERR_UNSUPPORTED;
  if (!q || !k || !v || !g || !beta || !o || !cu_seqlens) return XK_ERR_INVALID;
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(o, 8))
    return XK_ERR_INVALID;
  return XK_OK;
}

}  // namespace
}  // namespace xk

extern "C" int xk_gdn_chunk_fwd(
    const void* q, const void* k, const void* v, xk_dtype dtype, const void* g,
    xk_dtype g_dtype, const void* beta, xk_dtype beta_dtype, void* o,
    const float* initial_state, float* final_state, const void* cu_seqlens,
    xk_dtype cu_dtype, int64_t N, int64_t total_tokens, int64_t H, int64_t HV,
    int64_t K, int64_t V, float scale, int use_qk_l2norm, void* workspace,
    size_t workspace_bytes, void* stream) {
  bool empty = false;
  const int ast = chunk_args_status(q, k, v, dtype, g, g_dtype, beta, beta_dtype, o, cu_seqlens,
                                    cu_dtype, N, total_tokens, H, HV, K, V, &empty);
  if (ast != XK_OK || empty) return ast;
  const int64_t need = xk_gdn_chunk_workspace_bytes(total_tokens, N, HV);
  if (!workspace || static_cast<int64_t>(workspace_bytes) < need) return XK_ERR_WORKSPACE;
  if (!aligned(workspace, 256)) return XK_ERR_WORKSPACE;
  ChunkParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.g = g;
  p.beta = beta;
  p.o = o;
  p.h0 = initial_state;
  p.ht = final_state;
  p.cu = cu_seqlens;
  p.cu_i64 = cu_dtype == XK_I64;
  char* ws = static_cast<char*>(workspace);
  p.chunk_off = reinterpret_cast<int32_t*>(ws);
  ws += align256(4 * (N + 1));
  p.seq_order = reinterpret_cast<int32_t*>(ws);
  ws += align256(4 * N);
  p.ctab = reinterpret_cast<int2*>(ws);
  ws += align256(8 * nt_max(total_tokens, N));
  p.dump = reinterpret_cast<bf16*>(ws);
  p.rec = ws + kDump;
  p.N = N;
  p.NTmax = nt_max(total_tokens, N);
  p.T = total_tokens;
  p.H = static_cast<int>(H);
  p.HV = static_cast<int>(HV);
  p.scale = scale;
  p.l2norm = use_qk_l2norm;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (g_dtype == XK_F32) return chunk_beta<128, float>(p, V, beta_dtype, s);
  return chunk_beta<128, bf16>(p, V, beta_dtype, s);
}

// ---------------------------------------------------------------------------
// xk_gdn_chunk_fwd_noalloc: the same pipeline with its workspace in a static
// device buffer.  Each GPU holds its own copy of `scratch` from the moment
// this code object is loaded on it until the process ends.  In host code the
// name `scratch` is only a handle for the runtime: the device address of a
// GPU's copy comes from hipGetSymbolAddress, called once per device with that
// device current, and only that address is handed to the kernels.  Every call
// rewrites the parts of the workspace it reads (chunk table, offsets,
// records) before reading them, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
namespace {

constexpr int64_t kNoAllocScratchBytes = int64_t{64} << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_addr[kMaxDevices];
std::mutex g_scratch_mu;

// Device address of the current device's `scratch` (looked up on the first
// call per device).  `stream` must belong to the current device.
int scratch_on_current_device(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return XK_ERR_UNSUPPORTED;
  hipDevice_t sdev = -1;
  e = hipStreamGetDevice(stream, &sdev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (sdev != dev) return XK_ERR_INVALID;
  void* addr = g_scratch_addr[dev].load(std::memory_order_acquire);
  if (!addr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    addr = g_scratch_addr[dev].load(std::memory_order_relaxed);
    if (!addr) {
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return static_cast<int>(e);
      if (!addr) return XK_ERR_UNSUPPORTED;
      g_scratch_addr[dev].store(addr, std::memory_order_release);
    }
  }
  *out = addr;
  return XK_OK;
}

}  // namespace

extern "C" int xk_gdn_chunk_fwd_noalloc(
    const void* q, const void* k, const void* v, xk_dtype dtype, const void* g,
    xk_dtype g_dtype, const void* beta, xk_dtype beta_dtype, void* o,
    const float* initial_state, float* final_state, const void* cu_seqlens,
    xk_dtype cu_dtype, int64_t N, int64_t total_tokens, int64_t H, int64_t HV,
    int64_t K, int64_t V, float scale, int use_qk_l2norm, void* stream) {
  // The same argument checks as xk_gdn_chunk_fwd, before the size check.
  bool empty = false;
  const int ast = chunk_args_status(q, k, v, dtype, g, g_dtype, beta, beta_dtype, o, cu_seqlens,
                                    cu_dtype, N, total_tokens, H, HV, K, V, &empty);
  if (ast != XK_OK || empty) return ast;
  const int64_t need = xk_gdn_chunk_workspace_bytes(total_tokens, N, HV);
  if (need < 0) return XK_ERR_INVALID;
  if (need > kNoAllocScratchBytes) return XK_ERR_SCRATCH;
  void* ws = nullptr;
  const int st = scratch_on_current_device(static_cast<hipStream_t>(stream), &ws);
  if (st != XK_OK) return st;
  return xk_gdn_chunk_fwd(q, k, v, dtype, g, g_dtype, beta, beta_dtype, o, initial_state,
                          final_state, cu_seqlens, cu_dtype, N, total_tokens, H, HV, K, V,
                          scale, use_qk_l2norm, ws, static_cast<size_t>(kNoAllocScratchBytes),
                          stream);
}
