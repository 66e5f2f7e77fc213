// The chunked gated delta rule as separate stages (cumsum .. output), each with the
// tensor layout of the reference stage it replaces, for callers that drive
// the pipeline stage by stage (triton_npu/torch_api/triton_ops_api.h:34-66,
// 124-135).  The fused xk_gdn_chunk_fwd computes the same result in three
// launches without these intermediates.
//
// Layouts (rows = tokens of all sequences, cu_seqlens gives the sequences;
// chunks of 64 tokens restart at every sequence start):
//   g, g_cumsum, beta  [T, H]          k, q  [T, Hg, K]     v, u, v_new, o [T, H, V]
//   A, Ai              [T, H, 64]      w     [T, H, K]      h [NT, H, K, V]
// where row t of A / Ai holds row (t - chunk start) of that chunk's 64x64
// matrix and NT counts the chunks of all sequences in order.
//
// Stage semantics (fp32 arithmetic; decays are exp(x) for x <= 0, else 0):
//   cumsum   g_cumsum = per-chunk inclusive cumsum of g           (cumsum.py)
//   kkt      A[i][j] = b_i (k_i . k_j) exp(gc_i - gc_j), i > j     (chunk_scaled_dot_kkt.py:20-86)
//   solve    Ai = (I + A)^-1                                       (solve_tril.py)
//   w_u      u = Ai (v b),  w = Ai (k b exp(gc))                   (wy_fast.py:21-87)
//   fwd_h    per chunk: h_c = S;  v_new = u - w S;
//            S <- exp(gc_last) S + k^T (v_new exp(gc_last - gc))    (chunk_delta_h.py:22-198)
//   fwd_o    o = scale (exp(gc) (q h_c) + tril(q k^T exp(gc_i - gc_j)) v_new)
//                                                                  (chunk_o.py:21-115)
#include "gdn_common.h"

namespace xk {
namespace {

using namespace gdn;

constexpr int kTh = 256;

// Common sequence fields (read by cu_at / locate_chunk / chunk_offsets_kernel).
struct Seq {
  const void* cu;
  int cu_i64;
  int64_t N;
  int64_t T;  // token rows
  int32_t* chunk_off;
  int32_t* seq_order;  // sequences, longest first (fwd_h), or NULL
  int64_t NTmax;
};

// ---------------------------------------------------------------------------
// Per-chunk cumsum.  Chunks longer than 64: one thread per (token, head)
// summing its chunk prefix.
// ---------------------------------------------------------------------------
struct CumsumParams : Seq {
  const void* g;
  float* out;
  int H;
  int chunk;
};

template <typename GT>
__global__ void __launch_bounds__(kTh) chunk_cumsum_kernel(CumsumParams p) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * kTh + threadIdx.x;
  if (idx >= p.T * p.H) return;
  const int64_t t = idx / p.H;
  const int h = static_cast<int>(idx - t * p.H);
  float acc = 0.f;
  if (t >= cu_at(p, 0) && t < cu_at(p, p.N)) {
    int64_t lo = 0, hi = p.N;  // cu[lo] <= t < cu[hi]
    while (hi - lo > 1) {
      const int64_t mid = (lo + hi) >> 1;
      if (cu_at(p, mid) <= t) lo = mid; else hi = mid;
    }
    const int64_t bos = cu_at(p, lo);
    const int64_t cs = bos + ((t - bos) / p.chunk) * p.chunk;
    for (int64_t j = cs; j <= t; ++j) acc += ldf<GT>(p.g, j * p.H + h);
  }
  p.out[idx] = acc;
}

// Chunk sizes up to 64: one wave per (64-token block, head).  Each lane
// loads one g, a segmented wave scan (segments = chunks) sums within the
// block, and the tokens of lane 0's chunk that precede the block (at most
// 63) are summed once and added to that chunk's lanes.  Every g is read
// about twice instead of up to 64 times, and cu_seqlens is searched in LDS
// (up to kScanLdsSeqs sequences) so no lane waits on a chain of global
// reads.
constexpr int64_t kScanLdsSeqs = 1023;

// Start of the sequence holding token t, or -1; cu(i) reads cu_seqlens.
template <class CU>
__device__ __forceinline__ int64_t seq_start_of(const Seq& p, int64_t t, CU cu) {
  if (t >= p.T || t < cu(0) || t >= cu(p.N)) return -1;
  int64_t lo = 0, hi = p.N;  // cu[lo] <= t < cu[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (cu(mid) <= t) lo = mid; else hi = mid;
  }
  return cu(lo);
}

template <typename GT>
__global__ void __launch_bounds__(kTh) chunk_cumsum_scan_kernel(CumsumParams p) {
  __shared__ int64_t scu[kScanLdsSeqs + 1];
  const bool small = p.N <= kScanLdsSeqs;
  if (small)
    for (int64_t i = threadIdx.x; i <= p.N; i += kTh) scu[i] = cu_at(p, i);
  __syncthreads();
  auto cu = [&](int64_t i) { return small ? scu[i] : cu_at(p, i); };
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t wv = static_cast<int64_t>(blockIdx.x) * (kTh / kWave) + (threadIdx.x >> 6);
  const int64_t tb = wv / p.H;
  const int h = static_cast<int>(wv - tb * p.H);
  const int64_t t0 = tb * kWave;
  if (t0 >= p.T) return;  // wave-uniform, after the block's only barrier
  const int64_t t = t0 + lane;
  const int64_t bos = seq_start_of(p, t, cu);
  const int64_t cs = bos >= 0 ? bos + ((t - bos) / p.chunk) * p.chunk : t;
  float x = bos >= 0 ? ldf<GT>(p.g, t * p.H + h) : 0.f;
  // Lane l's segment starts at lane max(cs - t0, 0); tokens outside every
  // sequence are segments of their own (and stay 0).
  const int seg0 = static_cast<int>(max<int64_t>(cs - t0, 0));
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const float y = __shfl_up(x, o, kWave);
    if (lane - o >= seg0) x += y;
  }
  const int64_t bos0 = seq_start_of(p, t0, cu);
  const int64_t cs0 = bos0 >= 0 ? bos0 + ((t0 - bos0) / p.chunk) * p.chunk : t0;
  float c = 0.f;
  if (cs0 + lane < t0) c = ldf<GT>(p.g, (cs0 + lane) * p.H + h);
  c = group_sum<kWave>(c);
  if (bos >= 0 && cs == cs0) x += c;
  if (t < p.T) p.out[t * p.H + h] = x;
}

// Chunk size 64, up to kTileMaxHeads heads and kScanLdsSeqs sequences: one
// block per chunk.  A chunk's g rows [s, s + L) x H are contiguous, so the
// block loads them with coalesced reads into an LDS tile, each wave scans
// whole heads down the tile (lane = token), and the block stores the tile
// back with coalesced writes: every g read once and every output written
// once.  The chunk_cumsum_scan_kernel layout (a wave per 64-token block and
// head) reads with a stride of H values between lanes and re-reads the
// prefix of a chunk that starts before its block: 5x the op's bytes in HBM
// traffic at the prefill shape (16384 tokens x 32 heads) on MI355X.  Blocks
// past the last chunk zero the tokens outside every sequence, 64 at a time,
// as the other kernels do.
constexpr int kTileMaxHeads = 64;

template <typename GT>
__global__ void __launch_bounds__(kTh) chunk_cumsum_tile_kernel(CumsumParams p) {
  __shared__ int64_t scu[kScanLdsSeqs + 1];
  __shared__ int32_t soff[kScanLdsSeqs + 1];
  __shared__ float tile[kC][kTileMaxHeads + 1];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1), wid = tid >> 6;
  for (int64_t i = tid; i <= p.N; i += kTh) scu[i] = cu_at(p, i);
  __syncthreads();
  // Chunks of sequence n (none for an empty or malformed, decreasing, entry).
  auto nchunks = [&](int64_t n) {
    const int64_t len = scu[n + 1] - scu[n];
    return static_cast<int32_t>(len > 0 ? (len + kC - 1) / kC : 0);
  };
  if (wid == 0) {
    // Chunk offsets: lane l sums the chunk counts of its run of sequences,
    // then an exclusive wave scan places the runs.
    const int64_t per = (p.N + kWave - 1) / kWave;
    const int64_t b0 = lane * per, b1 = min(p.N, b0 + per);
    int32_t sum = 0;
    for (int64_t n = b0; n < b1; ++n) sum += nchunks(n);
    int32_t incl = sum;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int32_t t = __shfl_up(incl, o, kWave);
      if (lane >= o) incl += t;
    }
    int32_t acc = incl - sum;
    for (int64_t n = b0; n < b1; ++n) {
      soff[n] = acc;
      acc += nchunks(n);
    }
    if (lane == kWave - 1) soff[p.N] = incl;
  }
  __syncthreads();
  const int H = p.H;
  const int64_t b = blockIdx.x;
  const int64_t total = soff[p.N];
  int64_t s;
  int L;
  bool zero = false;
  if (b < total) {
    int64_t lo = 0, hi = p.N;  // soff[lo] <= b < soff[hi]
    while (hi - lo > 1) {
      const int64_t mid = (lo + hi) >> 1;
      if (soff[mid] <= b) lo = mid; else hi = mid;
    }
    s = scu[lo] + (b - soff[lo]) * kC;
    L = static_cast<int>(min<int64_t>(kC, scu[lo + 1] - s));
  } else {
    // Tokens [0, cu[0]) and [cu[N], T) belong to no sequence.
    const int64_t z = b - total;
    const int64_t head_tiles = (scu[0] + kC - 1) / kC;
    if (z < head_tiles) {
      s = z * kC;
      L = static_cast<int>(min<int64_t>(kC, scu[0] - s));
    } else {
      s = scu[p.N] + (z - head_tiles) * kC;
      if (s >= p.T) return;  // whole block
      L = static_cast<int>(min<int64_t>(kC, p.T - s));
    }
    zero = true;
  }
  const int n_el = L * H;
  const GT* g = reinterpret_cast<const GT*>(p.g) + s * H;
  float* out = p.out + s * H;
  if (zero) {
    for (int i = tid; i < n_el; i += kTh) out[i] = 0.f;
    return;
  }
  for (int i = tid; i < n_el; i += kTh) tile[i / H][i % H] = to_f32(g[i]);
  __syncthreads();
  for (int h = wid; h < H; h += kTh / kWave) {
    float x = lane < L ? tile[lane][h] : 0.f;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const float y = __shfl_up(x, o, kWave);
      if (lane >= o) x += y;
    }
    if (lane < L) tile[lane][h] = x;
  }
  __syncthreads();
  for (int i = tid; i < n_el; i += kTh) out[i] = tile[i / H][i % H];
}

// ---------------------------------------------------------------------------
// Scaled K K^T: A = strict_tril(b_i (k_i . k_j) exp(gc_i - gc_j)).  One wave per
// (chunk, head); the four waves of a block take four heads.
// ---------------------------------------------------------------------------
struct KktParams : Seq {
  const void* k;
  const void* beta;
  const float* gcum;  // or NULL
  float* A;
  int H, Hg;
};

template <int K, typename BT>
__global__ void __launch_bounds__(kTh) chunk_kkt_kernel(KktParams p) {
  __shared__ float vec[4][2][kC];  // gc, beta per wave
  // Wave index in a scalar register: the exit below is a scalar branch, and
  // the DPP transposes (q4_to_a) run with every lane of the wave active.
  const int wid = wave_index(), lane = threadIdx.x & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  // Blocks take the head groups of one chunk before the next chunk, so
  // that the blocks in flight read whole token rows.
  const int hg4 = (p.H + 3) >> 2;
  const int h = static_cast<int>(blockIdx.x % hg4) * 4 + wid;
  int64_t n, s;
  int L;
  const bool found = find_chunk(p, blockIdx.x / hg4, n, s, L);
  if (!(h < p.H && found)) return;  // wave-uniform
  const int hq = h / (p.H / p.Hg);
  constexpr int KK = K / 32;
  // Key rows loaded quad-contiguously (q4_load; rows >= L repeat row L-1)
  // and made A operands in registers; both operands of K K^T carry the same
  // key order, so the products are unchanged.
  static_assert(K == 128, "q4 operand loads are 16 x 128");
  const bf16* kbase = reinterpret_cast<const bf16*>(p.k) + static_cast<int64_t>(hq) * K;
  const int64_t rs = static_cast<int64_t>(p.Hg) * K;
  bf8_t kop[4][KK];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
    q4_load([&](int r) { return kbase + (s + min(mi * 16 + r, L - 1)) * rs; }, kop[mi]);
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) q4_to_a(kop[mi]);
  const int lt = min(lane, L - 1);
  vec[wid][0][lane] = p.gcum ? p.gcum[(s + lt) * p.H + h] : 0.f;
  vec[wid][1][lane] = ldf<BT>(p.beta, (s + lt) * p.H + h);
  __builtin_amdgcn_wave_barrier();
  // K K^T is symmetric, so the MFMA of tile (nj, mi) holds tile (mi, nj)
  // transposed: lane (l15, lg) gets row mi*16 + l15, columns nj*16 + 4lg ..
  // + 3, stored as one 16-byte vector.
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    const int row = mi * 16 + l15;
    const float brow = vec[wid][1][row], grow = vec[wid][0][row];
#pragma unroll
    for (int nj = 0; nj < 4; ++nj) {
      f4_t a = {0.f, 0.f, 0.f, 0.f};
      if (nj <= mi) {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) a = mfma16(kop[nj][kk], kop[mi][kk], a);
      }
      f4_t val;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int col = nj * 16 + 4 * lg + i;
        float v = 0.f;
        if (row > col) {
          v = brow * a[i];
          if (p.gcum) v *= safe_exp(grow - vec[wid][0][col]);
        }
        val[i] = v;
      }
      if (row < L)
        *reinterpret_cast<f4_t*>(p.A + ((s + row) * p.H + h) * kC + nj * 16 + 4 * lg) = val;
    }
  }
}

// ---------------------------------------------------------------------------
// Triangular solve: Ai = (I + A)^-1 per chunk.  One wave per (chunk, head).
// ---------------------------------------------------------------------------
struct TrilParams : Seq {
  const float* A;
  void* Ai;
  int H;
};

template <typename OT>
__global__ void __launch_bounds__(kTh) solve_tril_kernel(TrilParams p) {
  __shared__ __align__(16) float lds[4][kC][kLd];
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // Blocks take the head groups of one chunk before the next chunk, so
  // that the blocks in flight read whole token rows.
  const int hg4 = (p.H + 3) >> 2;
  const int h = static_cast<int>(blockIdx.x % hg4) * 4 + wid;
  int64_t n, s;
  int L;
  const bool found = find_chunk(p, blockIdx.x / hg4, n, s, L);
  if (!(h < p.H && found)) return;  // wave-uniform
  float (*X)[kLd] = lds[wid];
  // Access j covers rows 8j .. 8j + 7 (lane: row 8j + lane / 8, columns
  // 8 (lane % 8) .. + 7), so every instruction moves whole rows.  Strictly
  // lower part only; rows >= L are zero.
  const int sr = lane >> 3, sc = (lane & 7) * 8;
#pragma unroll
  for (int j = 0; j < kC / 8; ++j) {
    const int row = 8 * j + sr;
    const float* src = p.A + ((s + min(row, L - 1)) * p.H + h) * kC + sc;
    const f4_t a0 = *reinterpret_cast<const f4_t*>(src);
    const f4_t a1 = *reinterpret_cast<const f4_t*>(src + 4);
    f4_t m0, m1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      m0[e] = (row < L && sc + e < row) ? a0[e] : 0.f;
      m1[e] = (row < L && sc + 4 + e < row) ? a1[e] : 0.f;
    }
    *reinterpret_cast<f4_t*>(&X[row][sc]) = m0;
    *reinterpret_cast<f4_t*>(&X[row][sc + 4]) = m1;
  }
  __builtin_amdgcn_wave_barrier();
  invert_unit_lower(X);
#pragma unroll
  for (int j = 0; j < kC / 8; ++j) {
    const int row = 8 * j + sr;
    if (row < L) {
      Vec<OT, 8> o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o.v[e] = from_f32<OT>(X[row][sc + e]);
      *reinterpret_cast<Vec<OT, 8>*>(reinterpret_cast<OT*>(p.Ai) + ((s + row) * p.H + h) * kC + sc) = o;
    }
  }
}

// ---------------------------------------------------------------------------
// WY recompute: u = Ai (v b), w = Ai (k b exp(gc)).
// ---------------------------------------------------------------------------
struct WuParams : Seq {
  const void* k;
  const void* v;
  const void* beta;
  const float* gcum;
  const void* Ai;
  void* w;
  void* u;
  int H, Hg;
};

constexpr int kLt = kC + 8;  // bf16 LDS row stride (144 B: 16-byte aligned)

// One block per (chunk, head); wave w owns tokens 16w .. 16w + 15 of both
// products.  The per-token factors are folded into Ai's columns,
// u = (Ai diag(b)) v and w = (Ai diag(b exp(gc))) k, so the right-hand
// sides are the raw bf16 rows: they go from HBM straight into LDS tiles by
// direct loads (no registers, no conversion), whole rows at a time like the
// chunk's Ai rows, and the block waits once for all of it (Ai through
// registers, a quad reading four rows: 129.0 -> 124.5 us at config 4 on
// MI355X).  The scaled Ai rows are split hi / lo in registers (fp32 to
// ~2^-16) and are the B operands of both products, formed transposed,
// out^T = rhs^T Ai'^T, so that a lane owns one token and (through
// kr_at_pair's column order) 8 consecutive columns of it: 16-byte stores.
// Factors of key tokens >= L are 0, so those rows of the tiles (copies of
// row L - 1) add nothing.  Ai is lower triangular, so waves 0 and 1 skip
// the key tokens 32 .. 63.
template <typename BT, typename AT>
__global__ void __launch_bounds__(kTh) recompute_w_u_kernel(WuParams p) {
  constexpr int D = 128;  // K = V = 128
  static_assert(D == kKrRow, "row tiles of 128 bf16");
  __shared__ __align__(16) __bf16 vt[kC * D];  // v rows (kr_off layout)
  __shared__ __align__(16) __bf16 kt[kC * D];  // k rows (kr_off layout)
  __shared__ __align__(16) AT at[kC * kC];     // Ai rows, 16-byte chunk c of row r at c ^ (r % CPR)
  __shared__ __align__(16) float fb[kC], fk[kC];
  constexpr int CE = 16 / static_cast<int>(sizeof(AT));  // Ai elements per 16-byte chunk
  constexpr int CPR = kC / CE;                           // chunks per Ai row
  constexpr int RPI = 64 / CPR;                          // Ai rows per 1 KB load
  // Blocks take the heads of one chunk before the next chunk, so that the
  // blocks in flight read whole token rows.
  const int h = static_cast<int>(blockIdx.x % p.H);
  int64_t n, s;
  int L;
  if (!find_chunk(p, blockIdx.x / p.H, n, s, L)) return;  // block-uniform
  const int hq = h / (p.H / p.Hg);
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  // Rows 16w + 4j + lane / 16 of both tiles, 1 KB per load; LDS chunk
  // lane % 16 of row r holds the row's chunk (lane % 16) ^ (r % 16).
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = wid * 16 + 4 * j + lg;
    const int64_t t = s + min(r, L - 1);
    const int c = l15 ^ (r & 15);
    dma16(reinterpret_cast<const bf16*>(p.v) + (t * p.H + h) * D + 8 * c, vt + (wid * 16 + 4 * j) * D);
    dma16(reinterpret_cast<const bf16*>(p.k) + (t * p.Hg + hq) * D + 8 * c, kt + (wid * 16 + 4 * j) * D);
  }
  // Ai rows 16w .. 16w + 15 whole (CPR lanes a row), likewise.
#pragma unroll
  for (int j = 0; j < 16 / RPI; ++j) {
    const int r = wid * 16 + RPI * j + lane / CPR;
    const int c = (lane % CPR) ^ (r % CPR);
    dma16(reinterpret_cast<const AT*>(p.Ai) + ((s + min(r, L - 1)) * p.H + h) * kC + CE * c,
          at + (wid * 16 + RPI * j) * kC);
  }
  const int tq = wid * 16 + l15;
  // The 64 token factors (lane = token), loaded last so that their wait
  // overlaps the loads above.  (Fetching them by shuffles instead, which
  // brings the LDS to 40 KB and four blocks per CU with bf16 Ai, measured
  // 128.1 against 124.5 us at config 4 on MI355X.)
  const int64_t ft = (s + min(lane, L - 1)) * p.H + h;
  const float bval = ldf<BT>(p.beta, ft);
  const float gval = p.gcum ? p.gcum[ft] : 0.f;
  if (wid == 0) {
    fb[lane] = lane < L ? bval : 0.f;
    fk[lane] = lane < L ? bval * __expf(gval) : 0.f;
  }
  dma_sync();  // tiles, Ai rows and factors

  // Ai row tq, keys 32 kk + 8 lg .. + 7 (B operand layout).
  float ai[2][8];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk)
#pragma unroll
    for (int h8 = 0; h8 < 8 / CE; ++h8) {
      const int c = (32 * kk + 8 * lg) / CE + h8;
      const AT* src = at + tq * kC + CE * (c ^ (tq % CPR));
      if constexpr (CE == 8) {
        load_vec_f32<AT, 8>(src, ai[kk]);
      } else {
        float t4[4];
        load_vec_f32<AT, 4>(src, t4);
#pragma unroll
        for (int e = 0; e < 4; ++e) ai[kk][4 * h8 + e] = t4[e];
      }
    }

  bf8_t uh[2], ul[2], wh[2], wl[2];
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const float* pb = fb + 32 * kk + 8 * lg;
    const float* pk = fk + 32 * kk + 8 * lg;
    alignas(16) float xb[8];
    alignas(16) float xk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xb[e] = ai[kk][e] * pb[e];
      xk[e] = ai[kk][e] * pk[e];
    }
    split8(xb, uh[kk], ul[kk]);
    split8(xk, wh[kk], wl[kk]);
  }
  const f4_t zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int prod = 0; prod < 2; ++prod) {
    const __bf16* tile = prod == 0 ? vt : kt;
    const bf8_t* bh = prod == 0 ? uh : wh;
    const bf8_t* bl = prod == 0 ? ul : wl;
    bf16* orow = reinterpret_cast<bf16*>(prod == 0 ? p.u : p.w) +
                 ((s + min(tq, L - 1)) * p.H + h) * D;
#pragma unroll
    for (int a = 0; a < D / 32; ++a) {
      f4_t acc0 = zero, acc1 = zero;
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        if (kk * 32 > wid * 16 + 15) continue;  // key tokens beyond the diagonal
        const bf8_t r0 = kr_at_pair(tile, a, 0, kk);  // rhs^T columns, tokens 32kk + 8lg ..
        const bf8_t r1 = kr_at_pair(tile, a, 1, kk);
        acc0 = mfma16(r0, bh[kk], acc0);
        acc0 = mfma16(r0, bl[kk], acc0);
        acc1 = mfma16(r1, bh[kk], acc1);
        acc1 = mfma16(r1, bl[kk], acc1);
      }
      if (tq < L) {
        Vec<bf16, 8> ov;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ov.v[i] = from_f32<bf16>(acc0[i]);
          ov.v[4 + i] = from_f32<bf16>(acc1[i]);
        }
        *reinterpret_cast<Vec<bf16, 8>*>(orow + 32 * a + 8 * lg) = ov;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The state recurrence with per-chunk state snapshots.  One 256-lane
// block per (sequence, head, 32-column V tile); the fp32 state lives in
// registers (wave w: K rows [32w, 32w+32)), its bf16 hi / lo copy in LDS.
// ---------------------------------------------------------------------------
constexpr int kBV = 32;

struct FwdHParams : Seq {
  const void* k;
  const void* w;
  const void* u;
  const float* gcum;  // or NULL
  const float* h0;    // or NULL
  void* h;            // [NT, H, K, V]
  void* vnew;         // or NULL
  float* ht;          // or NULL
  int64_t hcap;       // chunks h holds
  int H, Hg;
  int nvt;
};

template <int K>
struct __align__(16) FwdHSmem {
  __bf16 sb[2][kBV][K + 8];  // state hi / lo, transposed: sb[h][v][k]
  __bf16 kr[kC * K];         // chunk key rows (kr_off layout)
  __bf16 dt[2][kBV][kLt];    // decayed v_new transposed, hi / lo
  float gc[kC];
};

// One chunk's global operands for this lane, loaded a chunk ahead: key rows
// and w rows wave*16 + lane%16 (A layout), the lane's u row in A layout
// (select_op turns it into C layout) and, for lanes < 64, one token's gc.
template <int KK>
struct FwdHOps {
  bf8_t ka[KK];  // K and w rows wid*16.. as q4_load_b leaves them: K is stored
  bf8_t wa[KK];  // as it is into the key tile, q4_to_a makes w A operands with
                 // keys in q4_key order
  bf8_t ua;
  float gct;
};

template <int K>
__global__ void __launch_bounds__(kTh) chunk_fwd_h_kernel(FwdHParams p) {
  __shared__ FwdHSmem<K> sm;
  constexpr int KK = K / 32, M2 = K / 64;
  static_assert(K == 128, "q4 operand loads are 16 x 128");
  const int tid = threadIdx.x, wid = wave_index(), lane = tid & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  const int64_t bid = blockIdx.x;
  const int64_t r = bid >> 3;
  const int vt = static_cast<int>(r % p.nvt);
  const int64_t item = (r / p.nvt) * 8 + (bid & 7);  // same XCD for one (n, h)
  if (item >= p.N * p.H) return;
  // Items are dispatched longest sequence first: the longest chains start in
  // the first wave of resident blocks and shorter ones fill in behind them.
  int64_t n, c0;
  find_ranked_seq(p, item / p.H, n, c0);
  const int h = static_cast<int>(item % p.H);
  const int hq = h / (p.H / p.Hg);
  const int V = p.nvt * kBV, v0 = vt * kBV;
  const int64_t bos = cu_at(p, n), eos = cu_at(p, n + 1);
  // Chunks of this sequence, bounded by the snapshots h can hold (never
  // binding for a well-formed cu_seqlens).
  const int64_t nch = max<int64_t>(0, min<int64_t>((eos - bos + kC - 1) / kC, p.hcap - c0));
  f4_t sreg[M2][2];
#pragma unroll
  for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
    for (int nj = 0; nj < 2; ++nj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kr = wid * (K / 4) + m2 * 16 + 4 * lg + i;
        sreg[m2][nj][i] = p.h0 ? p.h0[((n * p.H + h) * K + kr) * V + v0 + nj * 16 + l15] : 0.f;
      }
  const int64_t krow = static_cast<int64_t>(p.Hg) * K;
  const int64_t wrow = static_cast<int64_t>(p.H) * K;
  const bf8_t sel[2] = {select_op(0), select_op(1)};
  // B operand picking, for output column n, slot 8 (n / 4) + n % 4: the first
  // four slots of each lane group, i.e. the rows of one 16-row result tile.
  bf8_t sel4;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    sel4[e] = static_cast<__bf16>(lg == (l15 >> 2) && e == (l15 & 3) ? 1.0f : 0.0f);
  // K and w rows quad-contiguously (q4_load_b; the A-layout loads made each
  // quad read 4 different rows).
  auto load_ops = [&](FwdHOps<KK>& o, int64_t ci) {
    const int64_t s = bos + ci * kC;
    const int L = static_cast<int>(min<int64_t>(kC, eos - s));
    const WaveRows wr = wave_rows(s, L, wid);
    q4_load_b(reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.k) + wr.row0 * krow +
                                            static_cast<int64_t>(hq) * K),
              static_cast<uint32_t>(2 * krow), wr.lw, o.ka);
    q4_load_b(reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.w) + wr.row0 * wrow +
                                            static_cast<int64_t>(h) * K),
              static_cast<uint32_t>(2 * wrow), wr.lw, o.wa);
    o.ua = *reinterpret_cast<const bf8_t*>(
        reinterpret_cast<const bf16*>(p.u) +
        ((s + min(wid * 16 + l15, L - 1)) * p.H + h) * static_cast<int64_t>(V) + v0 + 8 * lg);
    o.gct = p.gcum ? p.gcum[(s + min(tid & (kC - 1), L - 1)) * p.H + h] : 0.f;
  };

  // One chunk; `cur` holds its operands, `nxt` receives the next chunk's
  // (the last chunk loads itself again, so every load is unconditional).
  auto step = [&](FwdHOps<KK>& cur, FwdHOps<KK>& nxt, int64_t ci) {
    const int64_t s = bos + ci * kC;
    const int L = static_cast<int>(min<int64_t>(kC, eos - s));
    const int64_t cidx = c0 + ci;
    load_ops(nxt, min(ci + 1, nch - 1));
    // Snapshot of the state entering this chunk (bf16, the hi part), and its
    // bf16 hi / lo copy.
    bf16* hdst = reinterpret_cast<bf16*>(p.h) + (cidx * p.H + h) * static_cast<int64_t>(K) * V;
    Vec<__bf16, 4> shi[M2][2];
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
      for (int nj = 0; nj < 2; ++nj) {
        Vec<__bf16, 4> lo;
        split4(sreg[m2][nj], shi[m2][nj], lo);
        const int k0 = wid * (K / 4) + m2 * 16 + 4 * lg;
        *reinterpret_cast<Vec<__bf16, 4>*>(&sm.sb[0][nj * 16 + l15][k0]) = shi[m2][nj];
        *reinterpret_cast<Vec<__bf16, 4>*>(&sm.sb[1][nj * 16 + l15][k0]) = lo;
      }
    // The snapshot is stored row-major (V fastest) as 8-byte vectors: the
    // lane's two key tiles of column nj form an A operand (row = column
    // v0 + 16 nj + l15, key slots), and select_op MFMAs (exact) hand each
    // lane 4 consecutive columns of one key, kappa below.
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) {
      bf8_t a;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        a[i] = shi[0][nj].v[i];
        a[4 + i] = shi[1][nj].v[i];
      }
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const f4_t t = mfma16(a, sel[hh], f4_t{0.f, 0.f, 0.f, 0.f});
        // Lane (lg, l15) now holds key row kappa(l15) and columns 4 lg ..;
        // quad_rows regroups the lanes so each quad stores 32 contiguous
        // bytes of one key row.
        const int r = quad_row() + 16 * hh, g = r >> 3, e = r & 7;
        const int kr = wid * (K / 4) + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4);
        Vec<bf16, 4> o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o.v[i] = static_cast<bf16>(t[i]);
        *reinterpret_cast<u32x2*>(hdst + static_cast<int64_t>(kr) * V + v0 + nj * 16 + 4 * quad_col()) =
            quad_rows(__builtin_bit_cast(u32x2, o));
      }
    }
    store_kr_q4(sm.kr, cur.ka, wid);
    q4_to_a(cur.wa);
    if (tid < kC) sm.gc[tid] = cur.gct;
    __syncthreads();
    // WS = w S (hi / lo S) for rows wid*16.., then v_new = u - WS.
    f4_t ws[2] = {f4_t{0.f, 0.f, 0.f, 0.f}, f4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
#pragma unroll
      for (int nj = 0; nj < 2; ++nj) {
        const bf8_t sh = *reinterpret_cast<const bf8_t*>(&sm.sb[0][nj * 16 + l15][q4_key(kk, lg)]);
        const bf8_t sl = *reinterpret_cast<const bf8_t*>(&sm.sb[1][nj * 16 + l15][q4_key(kk, lg)]);
        ws[nj] = mfma16(cur.wa[kk], sh, ws[nj]);
        ws[nj] = mfma16(cur.wa[kk], sl, ws[nj]);
      }
    const float gl = sm.gc[L - 1];
#pragma unroll
    for (int nj = 0; nj < 2; ++nj) {
      const f4_t uc = mfma16(cur.ua, sel[nj], f4_t{0.f, 0.f, 0.f, 0.f});
      Vec<__bf16, 4> dh, dl;
      f4_t d;
      bf8_t vb = {};  // v_new (bf16) of this tile as an A operand, slots 0..3
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wid * 16 + 4 * lg + i;
        const float vn = uc[i] - ws[nj][i];
        vb[i] = static_cast<__bf16>(vn);
        const float dec = row < L ? (p.gcum ? safe_exp(gl - sm.gc[row]) : 1.f) : 0.f;
        d[i] = vn * dec;
      }
      if (p.vnew) {
        // Transposed by one MFMA so a lane holds 4 consecutive columns of
        // token 16 wid + l15 (an 8-byte store).  Rows >= L repeat row L-1
        // (their operands are clamped to it), so storing them at row L-1
        // rewrites the same values.
        const f4_t t = mfma16(vb, sel4, f4_t{0.f, 0.f, 0.f, 0.f});
        const int row = wid * 16 + quad_row();  // after quad_rows (quad-contiguous store)
        Vec<bf16, 4> o;
#pragma unroll
        for (int i = 0; i < 4; ++i) o.v[i] = static_cast<bf16>(t[i]);
        *reinterpret_cast<u32x2*>(reinterpret_cast<bf16*>(p.vnew) +
                                  ((s + min(row, L - 1)) * p.H + h) * static_cast<int64_t>(V) +
                                  v0 + nj * 16 + 4 * quad_col()) = quad_rows(__builtin_bit_cast(u32x2, o));
      }
      split4(d, dh, dl);
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.dt[0][nj * 16 + l15][wid * 16 + 4 * lg]) = dh;
      *reinterpret_cast<Vec<__bf16, 4>*>(&sm.dt[1][nj * 16 + l15][wid * 16 + 4 * lg]) = dl;
    }
    __syncthreads();
    // S <- exp(gl) S + K^T D.
    const float egl = p.gcum ? __expf(gl) : 1.f;
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2) {
      const int mi = wid * M2 + m2;
      bf8_t kA[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) kA[kk] = kr_at(sm.kr, mi, kk);
#pragma unroll
      for (int nj = 0; nj < 2; ++nj) {
        f4_t acc = sreg[m2][nj];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] *= egl;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf8_t dh = *reinterpret_cast<const bf8_t*>(&sm.dt[0][nj * 16 + l15][kk * 32 + 8 * lg]);
          const bf8_t dl = *reinterpret_cast<const bf8_t*>(&sm.dt[1][nj * 16 + l15][kk * 32 + 8 * lg]);
          acc = mfma16(kA[kk], dh, acc);
          acc = mfma16(kA[kk], dl, acc);
        }
        sreg[m2][nj] = acc;
      }
    }
    __syncthreads();  // sb / kr / dt / gc are rewritten by the next chunk
  };
  FwdHOps<KK> opsA, opsB;
  if (nch > 0) load_ops(opsA, 0);
  // Unrolled by two so the operand buffers swap roles without copies.
  for (int64_t ci = 0; ci < nch; ci += 2) {
    step(opsA, opsB, ci);
    if (ci + 1 < nch) step(opsB, opsA, ci + 1);
  }
  if (p.ht) {
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
      for (int nj = 0; nj < 2; ++nj)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kr = wid * (K / 4) + m2 * 16 + 4 * lg + i;
          p.ht[((n * p.H + h) * K + kr) * V + v0 + nj * 16 + l15] = sreg[m2][nj][i];
        }
  }
}

// ---------------------------------------------------------------------------
// The state recurrence for V a multiple of 64: one 512-lane block per
// (sequence, head, 64-column V tile).  Wave (wr, cg) owns tokens 16 wr ..
// of v_new, state key rows 32 wr .. and columns cb = 32 cg .. of the tile
// (the fp32 state in registers, MFMA C layout).  What leaves for global
// memory is formed so that a lane holds 8 consecutive columns of one row
// (16-byte stores):
//   v_new^T = u^T - S^T w^T  (A: state-copy rows, in an order that pairs
//                             the two C tiles of a lane; B: w rows)
//   h snapshot               (the state copy's hi part read transposed)
// and D = v_new * decay goes to LDS as token rows, read transposed as the B
// operand of S <- exp(gl) S + K^T D.  Two barriers per chunk.  A chunk's
// operands are loaded two chunks ahead into registers (key and w rows
// whole, 16 lanes a row); its key and w rows go to LDS at the end of the
// chunk before, so each load has a whole chunk to land before anything
// waits for it.
// ---------------------------------------------------------------------------
constexpr int kTh8 = 512;

template <int K>
struct __align__(16) FwdH8Smem {
  __bf16 sb[2][64 * K];   // state hi / lo, transposed [v][k] (sb8_off)
  __bf16 kr[2][kC * K];   // chunk key rows (kr_off), double-buffered
  __bf16 wt[kC * K];      // chunk w rows (kr_off)
  __bf16 dt[2][kC * 64];  // D hi / lo, [token][v] (t8_off)
};

struct FwdH8Ops {
  bf8_t kraw[2], wraw[2];  // key / w rows 16 wr + 8 cg + 4 j + lane / 16, chunk lane % 16
  bf8_t ut;                // u of token 16 wr + lane % 16, columns cb + 8 (lane / 16) .. + 7
  float gct;               // gc of that token
  float gl;                // gc of the chunk's last token
};
// The register operands of a chunk, computed from its FwdH8Ops at the end of
// the chunk before (where that chunk's loads are waited for anyway), so the
// chunk itself reads no load destination: the compiler's memory-counter
// waits at a loop-carried load were conservative and held up the chunk.
struct FwdH8Carry {
  float u[8];  // ut as fp32
  float dg;    // gl - gct
  float egl;   // exp(gl)
};

// VN: v_new is written.
template <int K, bool VN>
__global__ void __launch_bounds__(kTh8) chunk_fwd_h8_kernel(FwdHParams p) {
  static_assert(K == 128, "key rows of 128");
  __shared__ FwdH8Smem<K> sm;
  constexpr int KK = K / 32, M2 = K / 64, NJ = 2;
  const int tid = threadIdx.x, wid = wave_index(), lane = tid & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  // Waves w and w + 4 share a SIMD and take token rows wr and 3 - wr.
  const int cg = wid >> 2, wr = cg ? 3 - (wid & 3) : (wid & 3), cb = 32 * cg;
  const int rl = lane >> 4, ch = lane & 15;  // whole-row loads: row in a load, 16-byte chunk
  const int64_t bid = blockIdx.x;
  const int64_t r = bid >> 3;
  const int vt = static_cast<int>(r % p.nvt);
  const int64_t item = (r / p.nvt) * 8 + (bid & 7);  // one XCD for the V tiles of (n, h)
  if (item >= p.N * p.H) return;
  int64_t n, c0;
  find_ranked_seq(p, item / p.H, n, c0);  // longest sequences first
  const int h = state_head(static_cast<int>(item % p.H), p.H, p.Hg);
  const int hq = h / (p.H / p.Hg);
  const int V = p.nvt * 64, v0 = vt * 64;
  const int64_t bos = cu_at(p, n), eos = cu_at(p, n + 1);
  // Chunk counters are 32-bit (scalar compares; a sequence has < 2^31 chunks).
  const int nch = static_cast<int>(max<int64_t>(0, min<int64_t>((eos - bos + kC - 1) / kC, p.hcap - c0)));

  f4_t sreg[M2][NJ];
#pragma unroll
  for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
    for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kr = wr * (K / 4) + m2 * 16 + 4 * lg + i;
        sreg[m2][nj][i] = p.h0 ? p.h0[((n * p.H + h) * K + kr) * V + v0 + cb + nj * 16 + l15] : 0.f;
      }
  auto publish_state = [&]() {
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj) {
        Vec<__bf16, 4> hi, lo;
        split4(sreg[m2][nj], hi, lo);
        const int k0 = wr * (K / 4) + m2 * 16 + 4 * lg;
        *reinterpret_cast<Vec<__bf16, 4>*>(&sm.sb[0][sb8_off(cb + nj * 16 + l15, k0)]) = hi;
        *reinterpret_cast<Vec<__bf16, 4>*>(&sm.sb[1][sb8_off(cb + nj * 16 + l15, k0)]) = lo;
      }
  };
  const uint32_t krb = static_cast<uint32_t>(p.Hg) * K * 2;  // key row bytes
  const uint32_t wrb = static_cast<uint32_t>(p.H) * K * 2;   // w row bytes
  const int64_t vrow = static_cast<int64_t>(p.H) * V;         // u / v_new row elements
  const int vcol = h * V + v0 + cb + 8 * lg;                   // this lane's u / v_new columns
  auto load_ops = [&](FwdH8Ops& o, int ci) {
    const int64_t s = bos + static_cast<int64_t>(ci) * kC;
    const int L = static_cast<int>(min<int64_t>(kC, eos - s));
    const char* kb = reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.k) + (s * p.Hg + hq) * K);
    const char* wb = reinterpret_cast<const char*>(reinterpret_cast<const bf16*>(p.w) + (s * p.H + h) * K);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t row = static_cast<uint32_t>(min(wr * 16 + cg * 8 + 4 * j + rl, L - 1));
      o.kraw[j] = *reinterpret_cast<const bf8_t*>(kb + row * krb + 16u * ch);
      o.wraw[j] = *reinterpret_cast<const bf8_t*>(wb + row * wrb + 16u * ch);
    }
    const int64_t t = s + min(wr * 16 + l15, L - 1);
    o.ut = *reinterpret_cast<const bf8_t*>(reinterpret_cast<const bf16*>(p.u) + t * vrow + vcol);
    o.gct = p.gcum ? p.gcum[t * p.H + h] : 0.f;
    o.gl = p.gcum ? p.gcum[(s + L - 1) * p.H + h] : 0.f;
  };
  auto store_rows = [&](__bf16* tile, const bf8_t (&raw)[2]) {
#pragma unroll
    for (int j = 0; j < 2; ++j)
      *reinterpret_cast<bf8_t*>(tile + kr_off(wr * 16 + cg * 8 + 4 * j + rl, ch)) = raw[j];
  };

  // The empty asm statements pin the values here: without them the
  // conversions sink to their uses in the next chunk.
  auto carry = [&](FwdH8Carry& c, const FwdH8Ops& o) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      c.u[e] = static_cast<float>(o.ut[e]);
      asm volatile("" : "+v"(c.u[e]));
    }
    c.dg = o.gl - o.gct;
    c.egl = p.gcum ? __expf(o.gl) : 1.f;
    asm volatile("" : "+v"(c.dg), "+v"(c.egl));
  };
  FwdH8Ops opsA, opsB, opsC;
  FwdH8Carry cy;
  if (nch > 0) {
    load_ops(opsA, 0);
    load_ops(opsB, min(1, nch - 1));
    store_rows(sm.kr[0], opsA.kraw);
    store_rows(sm.wt, opsA.wraw);
    carry(cy, opsA);
  }
  publish_state();
  __syncthreads();

  // One chunk; `cy` holds its register operands, `mid` the next chunk's
  // operands (its rows go to LDS and its carry to `cy` at the end), `far`
  // receives the chunk after that (past the last chunk the last one loads
  // again, so every load is unconditional).
  auto step = [&](const FwdH8Ops& mid, FwdH8Ops& far, int ci) {
    const int64_t s = bos + static_cast<int64_t>(ci) * kC;
    const int L = static_cast<int>(min<int64_t>(kC, eos - s));
    const int64_t cidx = c0 + ci;
    load_ops(far, min(ci + 2, nch - 1));
    // (w S)^T: C tile hb holds columns cb + 8 lg + 4 hb + i of token 16 wr + l15.
    f4_t ws[2] = {f4_t{0.f, 0.f, 0.f, 0.f}, f4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const bf8_t wb = kr_a(sm.wt, wr, kk);
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        const int vr = cb + 8 * (l15 >> 2) + 4 * hb + (l15 & 3);
        const bf8_t sh = *reinterpret_cast<const bf8_t*>(&sm.sb[0][sb8_off(vr, kk * 32 + 8 * lg)]);
        const bf8_t sl = *reinterpret_cast<const bf8_t*>(&sm.sb[1][sb8_off(vr, kk * 32 + 8 * lg)]);
        ws[hb] = mfma16(sh, wb, ws[hb]);
        ws[hb] = mfma16(sl, wb, ws[hb]);
      }
    }
    const int tok = wr * 16 + l15;
    const float dec = tok < L ? (p.gcum ? safe_exp(cy.dg) : 1.f) : 0.f;
    alignas(16) float d[8];
    bf8_t vb;
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float vn = cy.u[4 * hb + i] - ws[hb][i];
        vb[4 * hb + i] = static_cast<__bf16>(vn);
        d[4 * hb + i] = vn * dec;
      }
    bf8_t dh, dl;
    split8(d, dh, dl);
    *reinterpret_cast<bf8_t*>(&sm.dt[0][t8_off(tok, cb + 8 * lg)]) = dh;
    *reinterpret_cast<bf8_t*>(&sm.dt[1][t8_off(tok, cb + 8 * lg)]) = dl;
    const float egl = cy.egl;
    __syncthreads();  // (1) D complete; state copy and w rows read

    // The chunk's global stores are issued here, beside the state update,
    // rather than in the chain before barrier (1): 240 -> 199 us at config 4
    // on MI355X.
    // Rows >= L repeat row L - 1 (their operands are clamped to it), so they
    // store the same values there: the store is unconditional (a store that
    // only some paths issue makes the compiler wait for every outstanding
    // prefetch, gfx9 counting loads and stores in one counter).
    if constexpr (VN)
      *reinterpret_cast<bf8_t*>(reinterpret_cast<bf16*>(p.vnew) + (s + min(tok, L - 1)) * vrow + vcol) = vb;
    // Snapshot of the state entering this chunk (its bf16 hi part, still in
    // the state copy until publish_state below): lane (lg, l15) stores key
    // 32 wr + 16 t + l15, columns cb + 8 lg .. + 7.
    bf16* hdst = reinterpret_cast<bf16*>(p.h) + (cidx * p.H + h) * static_cast<int64_t>(K) * V + v0 + cb + 8 * lg;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int kc = wr * 32 + 16 * t;
      const bf8_t x = cat_bf8(sb8_col4(sm.sb[0], kc, cb + 8 * lg), sb8_col4(sm.sb[0], kc, cb + 8 * lg + 4));
      *reinterpret_cast<bf8_t*>(hdst + static_cast<int64_t>(kc + l15) * V) = x;
    }
    // S <- exp(gl) S + K^T D for key rows 32 wr .., columns cb ...
    const __bf16* kr = sm.kr[ci & 1];
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
        for (int i = 0; i < 4; ++i) acc[i] *= egl;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const int r0 = kk * 32 + 8 * lg;
          const bf8_t xh = cat_bf8(t8_col4(sm.dt[0], cb + nj * 16, r0), t8_col4(sm.dt[0], cb + nj * 16, r0 + 4));
          const bf8_t xl = cat_bf8(t8_col4(sm.dt[1], cb + nj * 16, r0), t8_col4(sm.dt[1], cb + nj * 16, r0 + 4));
          acc = mfma16(ka[kk], xh, acc);
          acc = mfma16(ka[kk], xl, acc);
        }
        sreg[m2][nj] = acc;
      }
    }
    publish_state();
    store_rows(sm.kr[(ci + 1) & 1], mid.kraw);
    store_rows(sm.wt, mid.wraw);
    carry(cy, mid);
    __syncthreads();  // (2) state copy, next rows written; key rows and D read
  };
  // Unrolled by three so the operand buffers rotate without copies; the
  // loop body has no branches around steps (the compiler's memory-counter
  // waits then follow the rotation), the last one or two chunks follow it.
  int ci = 0;
  for (; ci + 2 < nch; ci += 3) {
    step(opsB, opsC, ci);
    step(opsC, opsA, ci + 1);
    step(opsA, opsB, ci + 2);
  }
  if (ci < nch) step(opsB, opsC, ci);
  if (ci + 1 < nch) step(opsC, opsA, ci + 1);
  if (p.ht) {
#pragma unroll
    for (int m2 = 0; m2 < M2; ++m2)
#pragma unroll
      for (int nj = 0; nj < NJ; ++nj)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int kr = wr * (K / 4) + m2 * 16 + 4 * lg + i;
          p.ht[((n * p.H + h) * K + kr) * V + v0 + cb + nj * 16 + l15] = sreg[m2][nj][i];
        }
  }
}

// ---------------------------------------------------------------------------
// Output: o = scale (exp(gc) (q h_c) + tril(q k^T exp(gc_i - gc_j)) v_new).
// One block per (chunk, head): h_c and v_new staged transposed in LDS, wave
// w owns rows [16w, 16w+16) and all V columns.
// ---------------------------------------------------------------------------
struct FwdOParams : Seq {
  const void* q;
  const void* k;
  const void* v;
  const void* h;
  const float* gcum;  // or NULL
  void* o;
  float scale;
  int64_t hcap;  // chunks h holds
  int H, Hg;
};

template <int K, int V>
struct __align__(16) FwdOSmem {
  __bf16 hr[K * V];   // h_c rows hr[k][v] (kr_off layout)
  __bf16 vr[kC * V];  // v_new rows vr[token][v] (kr_off layout); rows >= L repeat row L - 1
  float gc[kC];
};

// One block per (chunk, head); wave w produces the outputs of tokens
// 16w .. 16w + 15.  Everything is computed transposed, o^T = h^T q^T +
// v^T Aq^T, so that a lane owns one token and 4 consecutive columns of it
// (one 8-byte store per 16 columns):
//  * h and v_new are loaded as whole rows and stored in LDS as they are;
//    their transposes are read with ds_read_b64_tr_b16 (kr_col4);
//  * Aq^T = (k q^T masked and decayed, rounded to bf16 as the reference's
//    A.to(v), chunk_o.py:113) stays in registers: its MFMA C layout holds 4
//    consecutive key tokens per lane, and two such tiles form the B operand
//    with the key tokens in the order {4g .. 4g+3, 16+4g .. 16+4g+3}; the
//    matching A operand reads the same tokens of v_new as two transposed
//    4-row reads.
// Three waves per SIMD (the LDS allows three blocks per CU) need at most
// 168 VGPRs: 166 with the cap against 172 without it, and the uncapped
// kernel (two waves per SIMD) took 205 us at config 4 on MI355X against 173.
template <int K, int V>
__global__ void __launch_bounds__(kTh) __attribute__((amdgpu_waves_per_eu(3)))
chunk_fwd_o_kernel(FwdOParams p) {
  static_assert(K == 128 && V == 128, "head dims of 128");
  __shared__ FwdOSmem<K, V> sm;
  constexpr int KK = K / 32, NJ = V / 16;
  const int tid = threadIdx.x, wid = wave_index(), lane = tid & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  // Heads of one chunk before the next chunk (whole token rows in flight).
  const int h = static_cast<int>(blockIdx.x % p.H);
  const int64_t c = blockIdx.x / p.H;
  int64_t n, s;
  int L;
  if (!find_chunk(p, c, n, s, L) || c >= p.hcap) return;  // block-uniform
  const int hq = h / (p.H / p.Hg);
  const f4_t zero = {0.f, 0.f, 0.f, 0.f};

  // Every global operand is loaded before its first use.  h and v_new rows
  // go straight into their LDS tiles by direct loads (1 KB = 4 whole rows a
  // load; LDS chunk lane % 16 of row r holds the row's chunk
  // (lane % 16) ^ (r % 16)); v_new rows >= L repeat row L - 1, which the
  // masked Aq multiplies by 0.  q and the key tiles of Aq follow in
  // registers.
  static_assert(V == kKrRow, "row tiles of 128 bf16");
  const int rl = lane >> 4, ch = lane & 15;  // row within a load, 16-byte chunk
  const bf16* hsrc = reinterpret_cast<const bf16*>(p.h) + (c * p.H + h) * static_cast<int64_t>(K) * V;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = wid * 32 + 4 * j + rl;
    dma16(hsrc + r * V + 8 * (ch ^ (r & 15)), sm.hr + (wid * 32 + 4 * j) * V);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = wid * 16 + 4 * j + rl;
    dma16(reinterpret_cast<const bf16*>(p.v) + ((s + min(t, L - 1)) * p.H + h) * static_cast<int64_t>(V) +
              8 * (ch ^ (t & 15)),
          sm.vr + (wid * 16 + 4 * j) * V);
  }
  const float gct = p.gcum ? p.gcum[(s + min(lane, L - 1)) * p.H + h] : 0.f;
  const int64_t qrow = static_cast<int64_t>(p.Hg) * K;
  const int tq = wid * 16 + l15;  // this lane's output token
  // q rows and the key rows of Aq, loaded quad-contiguously (q4_load; rows
  // >= L repeat row L-1) and made A operands in registers with the keys in
  // q4_key order, which every product below matches on its other side.
  static_assert(K == 128, "q4 operand loads are 16 x 128");
  const bf16* qbase = reinterpret_cast<const bf16*>(p.q) + static_cast<int64_t>(hq) * K;
  const bf16* kbase = reinterpret_cast<const bf16*>(p.k) + static_cast<int64_t>(hq) * K;
  bf8_t qa[KK], ka[4][KK];
  q4_load([&](int r) { return qbase + (s + min(wid * 16 + r, L - 1)) * qrow; }, qa);
  // Key tiles j <= w only (Aq is lower triangular).
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (j <= wid) q4_load([&](int r) { return kbase + (s + min(j * 16 + r, L - 1)) * qrow; }, ka[j]);
  if (wid == 0) sm.gc[lane] = gct;
  dma_sync();
  q4_to_a(qa);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (j <= wid) q4_to_a(ka[j]);

  const float gq = sm.gc[tq];

  // Aq^T tiles (key tokens 16j + 4lg + i, query token tq), j <= w.
  f4_t at[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    at[j] = zero;
    if (j <= wid) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) at[j] = mfma16(ka[j][kk], qa[kk], at[j]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tk = j * 16 + 4 * lg + i;
        const bool keep = tk <= tq && tq < L;
        at[j][i] = keep ? at[j][i] * (p.gcum ? safe_exp(gq - sm.gc[tk]) : 1.f) : 0.f;
      }
    }
  }
  // B operands: key tokens {32m + 4lg .. +3, 32m + 16 + 4lg .. +3}, bf16.
  bf8_t aqb[2];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      aqb[m][i] = static_cast<__bf16>(at[2 * m][i]);
      aqb[m][4 + i] = static_cast<__bf16>(at[2 * m + 1][i]);
    }

  const float eg = p.gcum ? __expf(gq) : 1.f;
  bf16* orow = reinterpret_cast<bf16*>(p.o) + ((s + min(tq, L - 1)) * p.H + h) * static_cast<int64_t>(V);
#pragma unroll
  for (int nj = 0; nj < NJ; ++nj) {
    f4_t acc = zero;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) acc = mfma16(kr_at_q4(sm.hr, nj, kk), qa[kk], acc);
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] *= eg;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      if (m * 32 > wid * 16 + 15) continue;  // key tokens beyond the diagonal
      const bf8_t va = cat_bf8(kr_col4(sm.vr, nj, m * 32 + 4 * lg),
                               kr_col4(sm.vr, nj, m * 32 + 16 + 4 * lg));
      acc = mfma16(va, aqb[m], acc);
    }
    if (tq < L) {
      Vec<bf16, 4> ov;
#pragma unroll
      for (int i = 0; i < 4; ++i) ov.v[i] = from_f32<bf16>(p.scale * acc[i]);
      *reinterpret_cast<Vec<bf16, 4>*>(orow + nj * 16 + 4 * lg) = ov;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
int seq_init(Seq& q, const void* cu, xk_dtype cu_dtype, int64_t N, int64_t T, void* ws,
             size_t ws_bytes, bool need_offsets) {
  if (N < 0 || T < 0) return XK_ERR_INVALID;
  if (cu_dtype != XK_I32 && cu_dtype != XK_I64) return XK_ERR_UNSUPPORTED;
  q.cu = cu;
  q.cu_i64 = cu_dtype == XK_I64;
  q.N = N;
  q.T = T;
  q.NTmax = T / kC + N;
  q.chunk_off = nullptr;
  q.seq_order = nullptr;
  if (need_offsets) {
    if (!ws || static_cast<int64_t>(ws_bytes) < align256(4 * (N + 1)) + align256(4 * N) ||
        !aligned(ws, 256))
      return XK_ERR_WORKSPACE;
    q.chunk_off = static_cast<int32_t*>(ws);
    q.seq_order = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + align256(4 * (N + 1)));
  }
  return XK_OK;
}

// Chunk offsets, and with `order` the longest-first ranking of the
// sequences into p.seq_order.
template <class P>
int launch_offsets(const P& p, hipStream_t s, bool order = false) {
  if (p.N <= kWaveSeqs) return XK_OK;  // the kernels look chunks up themselves
  hipLaunchKernelGGL(chunk_offsets_kernel<P>, dim3(1), dim3(256), 0, s, p,
                     order ? p.seq_order : nullptr, nullptr, int64_t{0});
  return launch_status();
}

}  // namespace
}  // namespace xk

using namespace xk;
using namespace xk::gdn;

extern "C" int64_t xk_gdn_stage_workspace_bytes(int64_t num_seqs) {
  if (num_seqs < 0) return -1;
  return align256(4 * (num_seqs + 1)) + align256(4 * num_seqs);
}

extern "C" int xk_chunk_local_cumsum(const void* g, xk_dtype g_dtype, float* out,
                                     int64_t total_tokens, int64_t H, const void* cu_seqlens,
                                     xk_dtype cu_dtype, int64_t N, int64_t chunk_size,
                                     void* stream) {
  CumsumParams p{};
  int st = seq_init(p, cu_seqlens, cu_dtype, N, total_tokens, nullptr, 0, false);
  if (st) return st;
  if (H <= 0 || chunk_size <= 0 || (chunk_size & (chunk_size - 1))) return XK_ERR_INVALID;
  if (total_tokens == 0) return XK_OK;
  if (!g || !out || !cu_seqlens) return XK_ERR_INVALID;
  p.g = g;
  p.out = out;
  p.H = static_cast<int>(H);
  p.chunk = static_cast<int>(chunk_size);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (chunk_size == kC && H <= kTileMaxHeads && N <= kScanLdsSeqs) {
    // One block per chunk (at most T / 64 + N), then the tiles of tokens
    // outside every sequence (at most T / 64 + 2 more, less the chunks).
    const int64_t blocks = cdiv(total_tokens, kC) + N + 2;
    switch (g_dtype) {
      case XK_F32: hipLaunchKernelGGL(chunk_cumsum_tile_kernel<float>, dim3(blocks), dim3(kTh), 0, s, p); break;
      case XK_BF16: hipLaunchKernelGGL(chunk_cumsum_tile_kernel<bf16>, dim3(blocks), dim3(kTh), 0, s, p); break;
      case XK_F16: hipLaunchKernelGGL(chunk_cumsum_tile_kernel<f16>, dim3(blocks), dim3(kTh), 0, s, p); break;
      default: return XK_ERR_UNSUPPORTED;
    }
    return launch_status();
  }
  if (chunk_size <= kC) {
    const int64_t blocks = cdiv(cdiv(total_tokens, kWave) * H, kTh / kWave);
    switch (g_dtype) {
      case XK_F32: hipLaunchKernelGGL(chunk_cumsum_scan_kernel<float>, dim3(blocks), dim3(kTh), 0, s, p); break;
      case XK_BF16: hipLaunchKernelGGL(chunk_cumsum_scan_kernel<bf16>, dim3(blocks), dim3(kTh), 0, s, p); break;
      case XK_F16: hipLaunchKernelGGL(chunk_cumsum_scan_kernel<f16>, dim3(blocks), dim3(kTh), 0, s, p); break;
      default: return XK_ERR_UNSUPPORTED;
    }
    return launch_status();
  }
  const int64_t blocks = cdiv(total_tokens * H, kTh);
  switch (g_dtype) {
    case XK_F32: hipLaunchKernelGGL(chunk_cumsum_kernel<float>, dim3(blocks), dim3(kTh), 0, s, p); break;
    case XK_BF16: hipLaunchKernelGGL(chunk_cumsum_kernel<bf16>, dim3(blocks), dim3(kTh), 0, s, p); break;
    case XK_F16: hipLaunchKernelGGL(chunk_cumsum_kernel<f16>, dim3(blocks), dim3(kTh), 0, s, p); break;
    default: return XK_ERR_UNSUPPORTED;
  }
  return launch_status();
}

extern "C" int xk_chunk_scaled_dot_kkt(const void* k, xk_dtype dtype, const void* beta,
                                       xk_dtype beta_dtype, const float* g_cumsum, float* A,
                                       int64_t total_tokens, int64_t Hg, int64_t H, int64_t K,
                                       const void* cu_seqlens, xk_dtype cu_dtype, int64_t N,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  KktParams p{};
  int st = seq_init(p, cu_seqlens, cu_dtype, N, total_tokens, workspace, workspace_bytes, true);
  if (st) return st;
  if (Hg <= 0 || H <= 0 || H % Hg) return XK_ERR_INVALID;
  if (dtype != XK_BF16 || K != 128) return XK_ERR_UNSUPPORTED;
  if (beta_dtype != XK_BF16 && beta_dtype != XK_F32) return XK_ERR_UNSUPPORTED;
  if (N == 0 || total_tokens == 0) return XK_OK;
  if (!k || !beta || !A || !cu_seqlens || !aligned(k, 16) || !aligned(A, 16))
    return XK_ERR_INVALID;
  p.k = k;
  p.beta = beta;
  p.gcum = g_cumsum;
  p.A = A;
  p.H = static_cast<int>(H);
  p.Hg = static_cast<int>(Hg);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((st = launch_offsets(p, s))) return st;
  const int64_t blocks = p.NTmax * ((H + 3) / 4);
  if (blocks > INT32_MAX) return XK_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<uint32_t>(blocks));
  if (beta_dtype == XK_BF16)
    hipLaunchKernelGGL((chunk_kkt_kernel<128, bf16>), grid, dim3(kTh), 0, s, p);
  else
    hipLaunchKernelGGL((chunk_kkt_kernel<128, float>), grid, dim3(kTh), 0, s, p);
  return launch_status();
}

extern "C" int xk_solve_tril(const float* A, void* Ai, xk_dtype ai_dtype, int64_t total_tokens,
                             int64_t H, const void* cu_seqlens, xk_dtype cu_dtype, int64_t N,
                             void* workspace, size_t workspace_bytes, void* stream) {
  TrilParams p{};
  int st = seq_init(p, cu_seqlens, cu_dtype, N, total_tokens, workspace, workspace_bytes, true);
  if (st) return st;
  if (H <= 0) return XK_ERR_INVALID;
  if (!is_float_dtype(ai_dtype)) return XK_ERR_UNSUPPORTED;
  if (N == 0 || total_tokens == 0) return XK_OK;
  if (!A || !Ai || !cu_seqlens || !aligned(A, 16) || !aligned(Ai, 16)) return XK_ERR_INVALID;
  p.A = A;
  p.Ai = Ai;
  p.H = static_cast<int>(H);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((st = launch_offsets(p, s))) return st;
  const int64_t blocks = p.NTmax * ((H + 3) / 4);
  if (blocks > INT32_MAX) return XK_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<uint32_t>(blocks));
  switch (ai_dtype) {
    case XK_F32: hipLaunchKernelGGL(solve_tril_kernel<float>, grid, dim3(kTh), 0, s, p); break;
    case XK_BF16: hipLaunchKernelGGL(solve_tril_kernel<bf16>, grid, dim3(kTh), 0, s, p); break;
    default: hipLaunchKernelGGL(solve_tril_kernel<f16>, grid, dim3(kTh), 0, s, p); break;
  }
  return launch_status();
}

extern "C" int xk_recompute_w_u(const void* k, const void* v, xk_dtype dtype, const void* beta,
                                xk_dtype beta_dtype, const float* g_cumsum, const void* Ai,
                                xk_dtype ai_dtype, void* w, void* u, int64_t total_tokens,
                                int64_t Hg, int64_t H, int64_t K, int64_t V,
                                const void* cu_seqlens, xk_dtype cu_dtype, int64_t N,
                                void* workspace, size_t workspace_bytes, void* stream) {
  WuParams p{};
  int st = seq_init(p, cu_seqlens, cu_dtype, N, total_tokens, workspace, workspace_bytes, true);
  if (st) return st;
  if (Hg <= 0 || H <= 0 || H % Hg) return XK_ERR_INVALID;
  if (dtype != XK_BF16 || K != 128 || V != 128) return XK_ERR_UNSUPPORTED;
  if (beta_dtype != XK_BF16 && beta_dtype != XK_F32) return XK_ERR_UNSUPPORTED;
  if (ai_dtype != XK_BF16 && ai_dtype != XK_F32) return XK_ERR_UNSUPPORTED;
  if (N == 0 || total_tokens == 0) return XK_OK;
  if (!k || !v || !beta || !Ai || !w || !u || !cu_seqlens) return XK_ERR_INVALID;
  if (!aligned(k, 16) || !aligned(v, 16) || !aligned(Ai, 16) || !aligned(w, 16) ||
      !aligned(u, 16))
    return XK_ERR_INVALID;
  p.k = k;
  p.v = v;
  p.beta = beta;
  p.gcum = g_cumsum;
  p.Ai = Ai;
  p.w = w;
  p.u = u;
  p.H = static_cast<int>(H);
  p.Hg = static_cast<int>(Hg);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((st = launch_offsets(p, s))) return st;
  if (p.NTmax * H > INT32_MAX) return XK_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<uint32_t>(p.NTmax * H));
  if (beta_dtype == XK_BF16) {
    if (ai_dtype == XK_BF16) hipLaunchKernelGGL((recompute_w_u_kernel<bf16, bf16>), grid, dim3(kTh), 0, s, p);
    else hipLaunchKernelGGL((recompute_w_u_kernel<bf16, float>), grid, dim3(kTh), 0, s, p);
  } else {
    if (ai_dtype == XK_BF16) hipLaunchKernelGGL((recompute_w_u_kernel<float, bf16>), grid, dim3(kTh), 0, s, p);
    else hipLaunchKernelGGL((recompute_w_u_kernel<float, float>), grid, dim3(kTh), 0, s, p);
  }
  return launch_status();
}

extern "C" int xk_chunk_fwd_h(const void* k, const void* w, const void* u, xk_dtype dtype,
                              const float* g_cumsum, const float* initial_state, void* h,
                              int64_t num_chunks, void* v_new, float* final_state,
                              int64_t total_tokens, int64_t Hg, int64_t H, int64_t K, int64_t V,
                              const void* cu_seqlens, xk_dtype cu_dtype, int64_t N,
                              void* workspace, size_t workspace_bytes, void* stream) {
  FwdHParams p{};
  int st = seq_init(p, cu_seqlens, cu_dtype, N, total_tokens, workspace, workspace_bytes, true);
  if (st) return st;
  if (Hg <= 0 || H <= 0 || H % Hg || num_chunks < 0) return XK_ERR_INVALID;
  p.hcap = num_chunks;
  if (dtype != XK_BF16 || K != 128 || V <= 0 || V % kBV) return XK_ERR_UNSUPPORTED;
  if (N == 0) return XK_OK;
  if (!k || !w || !u || !h || !cu_seqlens) return XK_ERR_INVALID;
  if (!aligned(k, 16) || !aligned(w, 16)) return XK_ERR_INVALID;
  p.k = k;
  p.w = w;
  p.u = u;
  p.gcum = g_cumsum;
  p.h0 = initial_state;
  p.h = h;
  p.vnew = v_new;
  p.ht = final_state;
  p.H = static_cast<int>(H);
  p.Hg = static_cast<int>(Hg);
  // 64-column tiles (16-byte accesses of u, v_new and h) where V and the
  // alignment allow, else 32-column tiles.
  const bool wide = V % 64 == 0 && aligned(u, 16) && aligned(h, 16) && aligned(v_new, 16);
  p.nvt = static_cast<int>(V / (wide ? 64 : kBV));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((st = launch_offsets(p, s, true))) return st;
  const int64_t blocks = cdiv(N * H, 8) * 8 * p.nvt;
  if (blocks > INT32_MAX) return XK_ERR_UNSUPPORTED;
  if (wide && v_new)
    hipLaunchKernelGGL((chunk_fwd_h8_kernel<128, true>), dim3(static_cast<uint32_t>(blocks)), dim3(kTh8), 0, s, p);
  else if (wide)
    hipLaunchKernelGGL((chunk_fwd_h8_kernel<128, false>), dim3(static_cast<uint32_t>(blocks)), dim3(kTh8), 0, s, p);
  else
    hipLaunchKernelGGL(chunk_fwd_h_kernel<128>, dim3(static_cast<uint32_t>(blocks)), dim3(kTh), 0, s, p);
  return launch_status();
}

extern "C" int xk_chunk_fwd_o(const void* q, const void* k, const void* v, const void* h,
                              int64_t num_chunks, xk_dtype dtype, const float* g_cumsum, void* o,
                              float scale, int64_t total_tokens, int64_t Hg, int64_t H,
                              int64_t K, int64_t V, const void* cu_seqlens, xk_dtype cu_dtype,
                              int64_t N, void* workspace, size_t workspace_bytes, void* stream) {
  FwdOParams p{};
  int st = seq_init(p, cu_seqlens, cu_dtype, N, total_tokens, workspace, workspace_bytes, true);
  if (st) return st;
  if (Hg <= 0 || H <= 0 || H % Hg || num_chunks < 0) return XK_ERR_INVALID;
  p.hcap = num_chunks;
  if (dtype != XK_BF16 || K != 128 || V != 128) return XK_ERR_UNSUPPORTED;
  if (N == 0 || total_tokens == 0) return XK_OK;
  if (!q || !k || !v || !h || !o || !cu_seqlens) return XK_ERR_INVALID;
  if (!aligned(q, 16) || !aligned(k, 16) || !aligned(v, 16) || !aligned(h, 16) ||
      !aligned(o, 8))
    return XK_ERR_INVALID;
  p.q = q;
  p.k = k;
  p.v = v;
  p.h = h;
  p.gcum = g_cumsum;
  p.o = o;
  p.scale = scale;
  p.H = static_cast<int>(H);
  p.Hg = static_cast<int>(Hg);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if ((st = launch_offsets(p, s))) return st;
  if (p.NTmax * H > INT32_MAX) return XK_ERR_UNSUPPORTED;
  hipLaunchKernelGGL((chunk_fwd_o_kernel<128, 128>), dim3(static_cast<uint32_t>(p.NTmax * H)),
                     dim3(kTh), 0, s, p);
  return launch_status();
}
