// Device building blocks shared by the chunked gated-delta-rule kernels
// (the fused prefill in gdn_chunk.hip and the per-stage kernels in
// gdn_stages.hip): 64-token chunk enumeration from cu_seqlens, bf16 MFMA
// helpers with hi/lo-split fp32 operands, and the blocked inverse of a
// 64x64 unit-lower-triangular matrix.
#pragma once

#include "xk_common.h"

namespace xk {
namespace gdn {

constexpr int kC = 64;       // chunk size
constexpr int kLd = kC + 4;  // fp32 LDS row stride: rows stay 16-byte aligned

typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));

// 16x16x32 bf16 MFMA.  Lane l holds A[l%16][8(l/16)+e], B[8(l/16)+e][l%16]
// and C[4(l/16)+i][l%16].
__device__ __forceinline__ f4_t mfma16(const bf8_t& a, const bf8_t& b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// x = hi + lo with hi = bf16(x), lo = bf16(x - hi): together ~16 mantissa
// bits, so hi/lo-split products on the bf16 matrix cores stay within
// ~2^-16 of fp32.
__device__ __forceinline__ void split(float x, __bf16& hi, __bf16& lo) {
  hi = static_cast<__bf16>(x);
  lo = static_cast<__bf16>(x - static_cast<float>(hi));
}

typedef float f2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));

// split() of two values at once, with the same results: one packed
// conversion rounds both hi values, a shift and a mask widen them back to
// fp32, and a second packed conversion rounds both remainders (about half
// the instructions of two scalar splits, and the outputs come out packed).
__device__ __forceinline__ void split2(float a, float b, bf2_t& hi, bf2_t& lo) {
  hi = __builtin_convertvector(f2_t{a, b}, bf2_t);
  const uint32_t u = __builtin_bit_cast(uint32_t, hi);
  const float ha = __builtin_bit_cast(float, u << 16);
  const float hb = __builtin_bit_cast(float, u & 0xffff0000u);
  lo = __builtin_convertvector(f2_t{a - ha, b - hb}, bf2_t);
}

// Four values (an MFMA C fragment) split into hi / lo bf16 quads.
__device__ __forceinline__ void split4(const f4_t& x, Vec<__bf16, 4>& h, Vec<__bf16, 4>& l) {
  bf2_t h0, l0, h1, l1;
  split2(x[0], x[1], h0, l0);
  split2(x[2], x[3], h1, l1);
  h.v[0] = h0[0];
  h.v[1] = h0[1];
  h.v[2] = h1[0];
  h.v[3] = h1[1];
  l.v[0] = l0[0];
  l.v[1] = l0[1];
  l.v[2] = l1[0];
  l.v[3] = l1[1];
}

// Eight consecutive fp32 values (16-byte aligned) split into hi / lo.
__device__ __forceinline__ void split8(const float* p, bf8_t& h, bf8_t& l) {
  const f4_t a = *reinterpret_cast<const f4_t*>(p);
  const f4_t b = *reinterpret_cast<const f4_t*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; e += 2) {
    bf2_t x, y;
    split2(a[e], a[e + 1], x, y);
    h[e] = x[0];
    h[e + 1] = x[1];
    l[e] = y[0];
    l[e + 1] = y[1];
    split2(b[e], b[e + 1], x, y);
    h[e + 4] = x[0];
    h[e + 5] = x[1];
    l[e + 4] = y[0];
    l[e + 5] = y[1];
  }
}

// B operand that selects columns 16h .. 16h + 15 of a 32-wide A operand:
// mfma16(a, select_op(h), 0) is that 16 x 16 block of A in C layout, so a
// lane that held 8 consecutive columns of one row (A layout) receives 4
// consecutive rows of one column -- a register transpose.  The products
// with 1 and the sums with 0 are exact.
__device__ __forceinline__ bf8_t select_op(int h) {
  const int lane = threadIdx.x & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  bf8_t b;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    b[e] = static_cast<__bf16>(8 * lg + e == l15 + 16 * h ? 1.0f : 0.0f);
  return b;
}

// ---------------------------------------------------------------------------
// Quad-contiguous loads of 16 x 128 MFMA A operands (bf16 rows of 128 keys).
// The A layout gives lane l row l % 16, so loading it directly makes the 4
// lanes of every quad read 4 different rows.  q4_load instead has each quad
// read 64 contiguous bytes (4 consecutive 8-key chunks of one row): load h,
// lane l = 16 g + 4 a + b holds row 4 a + h, chunk 4 g + b.  q4_to_a then
// transposes the 4 x 4 (load, lane-in-quad) blocks of every quad in
// registers (two DPP quad_perm stages), after which operand j, lane l holds
// row l % 16, chunk 4 (l / 16) + j: slot g of operand j is key chunk 4 g + j
// instead of 4 j + g.  Products over the keys are unchanged as long as the
// other operand reads its keys in that order.  Measured on the chunked
// state kernel (MI355X): quad-contiguous K and Q loads took it from 263 to
// 231 us (timing copies without the transpose).
// ---------------------------------------------------------------------------
template <typename RowPtr>
__device__ __forceinline__ void q4_load(RowPtr row, bf8_t (&r)[4]) {
  const int lane = threadIdx.x & 63;
  const int a = (lane >> 2) & 3, chunk = 4 * (lane >> 4) + (lane & 3);
#pragma unroll
  for (int h = 0; h < 4; ++h) r[h] = *reinterpret_cast<const bf8_t*>(row(4 * a + h) + 8 * chunk);
}

// q4_load with the rows given as a wave-uniform base, a row pitch of rb
// bytes (< 2^24) and rows past lw clamped to lw: each address is the base
// plus a 32-bit lane offset.
__device__ __forceinline__ void q4_load_b(const char* base, uint32_t rb, int lw, bf8_t (&r)[4]) {
  const int lane = threadIdx.x & 63;
  const int a = (lane >> 2) & 3, chunk = 4 * (lane >> 4) + (lane & 3);
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const uint32_t off = __umul24(static_cast<uint32_t>(min(4 * a + h, lw)), rb) + 16u * chunk;
    r[h] = *reinterpret_cast<const bf8_t*>(base + off);
  }
}

// The 16 rows of wave `wid` in a chunk starting at token s with L valid
// rows: rows past L - 1 repeat row L - 1.  Split into a wave-uniform first
// row (s + min(16 wid, L - 1)) and a per-lane row offset min(r, lw), lw =
// L - 1 - min(16 wid, L - 1) >= 0, so every load address is a scalar base
// plus a 32-bit lane offset (the saddr form of global loads): the 64-bit
// per-lane address arithmetic this replaces was ~200 VALU instructions per
// chunk step.
struct WaveRows {
  int64_t row0;  // first row (token index)
  int lw;        // last valid row offset from row0
};
__device__ __forceinline__ WaveRows wave_rows(int64_t s, int L, int wid) {
  const int f = min(16 * wid, L - 1);
  return {s + f, L - 1 - f};
}
// Byte offset of element e of row offset r (clamped to lw) in rows of `rb` bytes.
// (r <= 15 and rb < 2^24: a 24-bit multiply.)
__device__ __forceinline__ uint32_t row_off(int r, int lw, uint32_t rb, int e) {
  return __umul24(static_cast<uint32_t>(min(r, lw)), rb) + 2u * static_cast<uint32_t>(e);
}

// Quad-contiguous stores of MFMA-layout row pieces.  In the layouts that
// give lane (g = lane / 16, t = lane % 16) row t, columns 4 g .. 4 g + 3 (8
// bytes of bf16), the 4 lanes of a quad write 4 different rows.  quad_rows
// hands lane (r = lane / 16, a = lane / 4 % 4, b = lane % 4) the piece of
// row quad_row() = 4 a + r, column group quad_col() = b, read from lane
// 16 b + 4 a + r (ds_bpermute), so each quad writes 32 contiguous bytes of
// one row.  Every lane of the wave must be active.
__device__ __forceinline__ int quad_row() {
  const int lane = threadIdx.x & 63;
  return 4 * ((lane >> 2) & 3) + (lane >> 4);
}
__device__ __forceinline__ int quad_col() { return threadIdx.x & 3; }
__device__ __forceinline__ u32x2 quad_rows(u32x2 w) {
  const int lane = threadIdx.x & 63;
  const int src = 4 * (16 * (lane & 3) + 4 * ((lane >> 2) & 3) + (lane >> 4));  // byte address
  w[0] = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(w[0]));
  w[1] = __builtin_amdgcn_ds_bpermute(src, static_cast<int>(w[1]));
  return w;
}

// Wave index as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_index() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
}

template <int CTRL>
__device__ __forceinline__ bf8_t quad_dpp(const bf8_t& v) {
  typedef int i4_t __attribute__((ext_vector_type(4)));
  const i4_t u = __builtin_bit_cast(i4_t, v);
  i4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = __builtin_amdgcn_mov_dpp(u[i], CTRL, 0xF, 0xF, true);
  return __builtin_bit_cast(bf8_t, o);
}

// In place: register h, quad lane b -> register b, quad lane h.  Stage 1
// swaps the off-diagonal 2 x 2 blocks (lane ^ 2, register ^ 2), stage 2
// transposes each 2 x 2 block (lane ^ 1, register ^ 1).  Every DPP move is
// made by the whole wave before the selects: inside `c ? dpp(x) : y` the
// move is evaluated on one side of a branch only, under a partial EXEC,
// where it would read disabled lanes.
__device__ __forceinline__ void q4_to_a(bf8_t (&r)[4]) {
  const bool b0 = threadIdx.x & 1, b1 = (threadIdx.x >> 1) & 1;
  constexpr int kXor1 = 0xB1, kXor2 = 0x4E;  // quad_perm(1,0,3,2), (2,3,0,1)
  const bf8_t x0 = quad_dpp<kXor2>(r[0]), x1 = quad_dpp<kXor2>(r[1]);
  const bf8_t x2 = quad_dpp<kXor2>(r[2]), x3 = quad_dpp<kXor2>(r[3]);
  const bf8_t s0 = b1 ? x2 : r[0];
  const bf8_t s2 = b1 ? r[2] : x0;
  const bf8_t s1 = b1 ? x3 : r[1];
  const bf8_t s3 = b1 ? r[3] : x1;
  const bf8_t y0 = quad_dpp<kXor1>(s0), y1 = quad_dpp<kXor1>(s1);
  const bf8_t y2 = quad_dpp<kXor1>(s2), y3 = quad_dpp<kXor1>(s3);
  r[0] = b0 ? y1 : s0;
  r[1] = b0 ? s1 : y0;
  r[2] = b0 ? y3 : s2;
  r[3] = b0 ? s3 : y2;
}

// Key offset of slot g (lane / 16) of operand kk in q4_to_a's order.
__device__ __forceinline__ constexpr int q4_key(int kk, int g) { return 32 * g + 8 * kk; }

// ---------------------------------------------------------------------------
// A chunk's 64 x 128 bf16 key rows kept row-major in LDS and read both as
// rows (A operands of K S) and as columns (A operands of K^T X).  Rows are
// 256 bytes, unpadded; 16-byte chunk c of row r sits at chunk c ^ (r & 15),
// which keeps the raw quad-contiguous stores (store_kr_q4) and the row reads
// (kr_a) free of bank conflicts.
//
// Column reads use gfx950's ds_read_b64_tr_b16.  In each group of 16 lanes,
// element i (of 4) of lane j is element j % 4 of the 8 bytes that lane
// 4 i + j / 4 addressed (checked on MI355X with an index-valued tile).  So
// when lane s addresses row r0 + s / 4, columns c0 + 4 (s % 4) .. + 3, lane
// j receives column c0 + j at rows r0 .. r0 + 3: four consecutive k of an
// MFMA operand whose rows are the tile's columns.
// ---------------------------------------------------------------------------
constexpr int kKrRow = 128;  // bf16 per key row
__device__ __forceinline__ int kr_off(int r, int chunk) {
  return r * kKrRow + ((chunk ^ (r & 15)) << 3);
}

// The raw q4_load pieces of rows wid*16 .. wid*16 + 15 (load h: lane
// 16 g + 4 a + b holds row 4 a + h, chunk 4 g + b) into the tile.
__device__ __forceinline__ void store_kr_q4(__bf16* kr, const bf8_t (&r)[4], int wid) {
  const int lane = threadIdx.x & 63;
  const int a = (lane >> 2) & 3, chunk = 4 * (lane >> 4) + (lane & 3);
#pragma unroll
  for (int h = 0; h < 4; ++h)
    *reinterpret_cast<bf8_t*>(kr + kr_off(wid * 16 + 4 * a + h, chunk)) = r[h];
}

// A operand kk of rows wid*16 ..: lane row wid*16 + lane % 16, keys
// 32 kk + 8 (lane / 16) .. + 7.
__device__ __forceinline__ bf8_t kr_a(const __bf16* kr, int wid, int kk) {
  const int lane = threadIdx.x & 63;
  return *reinterpret_cast<const bf8_t*>(kr + kr_off(wid * 16 + (lane & 15), 4 * kk + (lane >> 4)));
}

// Column 16 mi + lane % 16 of the tile at rows r0 .. r0 + 3 (r0 may differ
// between the 16-lane groups, not within one), as 4 bf16 bit patterns.
typedef short s4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ s4_t kr_col4(const __bf16* kr, int mi, int r0) {
  typedef __attribute__((address_space(3))) s4_t lds_s4;
  const int s = threadIdx.x & 15;
  const int col = 16 * mi + 4 * (s & 3);
  const __bf16* p = kr + kr_off(r0 + (s >> 2), col >> 3) + (col & 7);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p));
}
__device__ __forceinline__ bf8_t cat_bf8(s4_t a, s4_t b) {
  return __builtin_bit_cast(bf8_t, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// A operand of the transpose: lane column (key) 16 mi + lane % 16, rows
// (tokens) 32 kk + 8 (lane / 16) .. + 7, as two transposed 4-row reads.
__device__ __forceinline__ bf8_t kr_at(const __bf16* kr, int mi, int kk) {
  const int r0 = 32 * kk + 8 * ((threadIdx.x & 63) >> 4);
  return cat_bf8(kr_col4(kr, mi, r0), kr_col4(kr, mi, r0 + 4));
}

// Transposed tiles of the state kernels have unpadded rows, 16-byte chunk c of row r
// stored at chunk c ^ (r & 15) (state copy: 128 keys, 16 chunks a row) or
// c ^ (r & 7) (64-token tiles, 8 chunks a row).  Their MFMA operand reads
// (ds_read_b128 of one chunk from 16 consecutive rows) then touch 16
// distinct chunks of each 256-byte bank line, which a probe on MI355X
// measured free of bank conflicts; padded rows of 272 / 144 bytes cost an
// extra cycle per 16 lanes.  The 8-byte stores of MFMA results keep one
// extra cycle per 16 lanes either way (stores take 128 bytes a cycle, and
// the 16 rows' half-chunks have one parity).
__device__ __forceinline__ int sb8_off(int r, int c) {
  return r * 128 + (((c >> 3) ^ (r & 15)) << 3) + (c & 7);
}
__device__ __forceinline__ int t8_off(int r, int c) {
  return r * 64 + (((c >> 3) ^ (r & 7)) << 3) + (c & 7);
}

// Column c0 + lane % 16 of a 64-wide t8_off tile at rows r0 .. r0 + 3 (c0 a
// multiple of 16 shared by a 16-lane group, r0 per group), as kr_col4.
__device__ __forceinline__ s4_t t8_col4(const __bf16* t, int c0, int r0) {
  typedef __attribute__((address_space(3))) s4_t lds_s4;
  const int s = threadIdx.x & 15;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(t + t8_off(r0 + (s >> 2), c0 + 4 * (s & 3))));
}
// Column c0 + lane % 16 of a 128-wide sb8_off tile at rows r0 .. r0 + 3.
__device__ __forceinline__ s4_t sb8_col4(const __bf16* t, int c0, int r0) {
  typedef __attribute__((address_space(3))) s4_t lds_s4;
  const int s = threadIdx.x & 15;
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(t + sb8_off(r0 + (s >> 2), c0 + 4 * (s & 3))));
}

// v-head of head slot c (item % HV) of the state kernels, whose blocks run
// on XCD c % 8.  With H a multiple of 8 the G = HV / H v-heads of one
// qk-head get slots of one XCD, so that their q / k reads meet in that
// XCD's L2 (at config 4 on MI355X the state kernel then reads q and k from
// HBM once instead of twice: 583 -> 451 MB fetched per call).
__device__ __forceinline__ int state_head(int c, int HV, int H) {
  if (H % 8 != 0) return c;
  const int G = HV / H, x = c & 7, q = c >> 3;
  return G * (x + 8 * (q / G)) + q % G;
}

// kr_at with the columns paired for 16-byte stores: lane (g, j) gets column
// 32 a + 8 (j / 4) + 4 hb + j % 4 at rows 32 kk + 8 g .. + 7 (each 16-lane
// group of a transposed read may address any four 4-column groups).  The C
// tiles of hb = 0 and 1 then give lane (g, j) columns 32 a + 8 g .. + 7 of
// row j of the product.
__device__ __forceinline__ bf8_t kr_at_pair(const __bf16* kr, int a, int hb, int kk) {
  typedef __attribute__((address_space(3))) s4_t lds_s4;
  const int lane = threadIdx.x & 63, s = lane & 15;
  const int r0 = 32 * kk + 8 * (lane >> 4) + (s >> 2);
  const __bf16* p0 = kr + kr_off(r0, 4 * a + (s & 3)) + 4 * hb;
  const __bf16* p1 = kr + kr_off(r0 + 4, 4 * a + (s & 3)) + 4 * hb;
  return cat_bf8(__builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p0)),
                 __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(p1)));
}

// Direct global -> LDS loads of 16 bytes per lane: lane l's bytes from `src`
// land at `lds` + 16 l (`lds` wave-uniform).  They count in vmcnt, and a
// workgroup barrier alone does not wait for them, so dma_sync waits for
// every outstanding load first (as the builtin, so that the compiler knows
// they are complete and adds no wait of its own later).
typedef __attribute__((address_space(3))) void lds_void;
__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds, 16, 0, 0);
}
__device__ __forceinline__ void dma_sync() {
  __builtin_amdgcn_s_waitcnt(0);  // vmcnt, expcnt and lgkmcnt all 0
  __syncthreads();
}

// kr_at with the rows in q4_to_a's key order: rows q4_key(kk, lane / 16)
// .. + 7, the partner of an operand kk that went through q4_to_a.
__device__ __forceinline__ bf8_t kr_at_q4(const __bf16* kr, int mi, int kk) {
  const int r0 = 32 * ((threadIdx.x & 63) >> 4) + 8 * kk;
  return cat_bf8(kr_col4(kr, mi, r0), kr_col4(kr, mi, r0 + 4));
}

// (ah + al)(bh + bl) without the lo*lo term.
__device__ __forceinline__ f4_t mfma_split3(const bf8_t& ah, const bf8_t& al, const bf8_t& bh,
                                            const bf8_t& bl, f4_t c) {
  c = mfma16(ah, bh, c);
  c = mfma16(ah, bl, c);
  return mfma16(al, bh, c);
}

template <typename T>
__device__ __forceinline__ float ldf(const void* p, int64_t i) {
  return to_f32(reinterpret_cast<const T*>(p)[i]);
}

// exp(x) for x <= 0, else 0 (the masked decay of the chunk kernels,
// triton_npu/triton_src/chunk_gated_delta_rule/utils.py:82-83).
__device__ __forceinline__ float safe_exp(float x) { return x <= 0.f ? __expf(x) : 0.f; }

// ---------------------------------------------------------------------------
// Sequences and chunks.  P provides cu (int32 or int64 [N+1], cu_i64), N,
// T (token rows) and chunk_off (int32 [N+1] device workspace).
// ---------------------------------------------------------------------------

// cu_seqlens[i], clamped to [0, T] so that a malformed table can never index
// past the token rows (or a workspace sized from T).
template <class P>
__device__ __forceinline__ int64_t cu_at(const P& p, int64_t i) {
  const int64_t v = p.cu_i64 ? reinterpret_cast<const int64_t*>(p.cu)[i]
                             : static_cast<int64_t>(reinterpret_cast<const int32_t*>(p.cu)[i]);
  return min(max(v, int64_t{0}), p.T);
}

// Chunks of sequence n (ceil(len / 64); 0 for an empty sequence).
template <class P>
__device__ __forceinline__ int32_t seq_chunks(const P& p, int64_t n) {
  const int64_t len = cu_at(p, n + 1) - cu_at(p, n);
  return static_cast<int32_t>(len > 0 ? (len + kC - 1) / kC : 0);
}

// Sequences whose count is at most this are ranked longest-first by
// chunk_offsets_kernel (an O(N^2 / 256) ranking); longer lists keep their
// own order.
constexpr int64_t kSortMaxSeqs = 2048;

// chunk_off[n] = sum_{m<n} ceil(len_m / 64), chunk_off[N] = total chunks.
// If `order` is given, order[r] = the sequence of rank r when sequences are
// sorted by chunk count, longest first (ties by index), or order[r] = r for
// more than kSortMaxSeqs sequences.  If `table` is given (ntab entries),
// table[c] = (first token, length) of global chunk c, (0, 0) past the last
// chunk; token indices must fit in int32.  One block of 256 threads.
template <class P>
__global__ void __launch_bounds__(256) chunk_offsets_kernel(P p, int32_t* order, int2* table,
                                                            int64_t ntab) {
  constexpr int kT = 256;
  __shared__ int32_t part[kT / kWave];
  // Up to kSortMaxSeqs sequences, cu_seqlens and the offsets are also kept
  // in LDS, so the table and ranking passes make no dependent global reads.
  __shared__ int64_t scu[kSortMaxSeqs + 1];
  __shared__ int32_t soff[kSortMaxSeqs + 1];
  const int tid = threadIdx.x;
  const bool small = p.N <= kSortMaxSeqs;
  if (small)
    for (int64_t i = tid; i <= p.N; i += kT) scu[i] = cu_at(p, i);
  __syncthreads();
  auto cuv = [&](int64_t i) { return small ? scu[i] : cu_at(p, i); };
  auto nchunks = [&](int64_t n) {
    const int64_t len = cuv(n + 1) - cuv(n);
    return static_cast<int32_t>(len > 0 ? (len + kC - 1) / kC : 0);
  };
  const int64_t per = (p.N + kT - 1) / kT;
  const int64_t b0 = tid * per, b1 = min(p.N, b0 + per);
  int32_t s = 0;
  for (int64_t n = b0; n < b1; ++n) s += nchunks(n);
  // Exclusive scan of the per-thread counts: wave64 shuffle scans, then the
  // four wave totals through LDS.
  const int lane = tid & (kWave - 1), wid = tid / kWave;
  int32_t incl = s;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int32_t t = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += t;
  }
  if (lane == kWave - 1) part[wid] = incl;
  __syncthreads();
  int32_t acc = incl - s;
  for (int w = 0; w < wid; ++w) acc += part[w];
  for (int64_t n = b0; n < b1; ++n) {
    p.chunk_off[n] = acc;
    if (small) soff[n] = acc;
    acc += nchunks(n);
  }
  if (tid == kT - 1) {
    p.chunk_off[p.N] = acc;
    if (small) soff[p.N] = acc;
  }
  __syncthreads();  // offsets complete and visible to the block
  auto offv = [&](int64_t i) { return small ? soff[i] : p.chunk_off[i]; };
  if (table) {
    const int64_t total = offv(p.N);
    for (int64_t c = tid; c < ntab; c += kT) {
      int2 e = make_int2(0, 0);
      if (c < total) {
        int64_t lo = 0, hi = p.N;  // off[lo] <= c < off[hi]
        while (hi - lo > 1) {
          const int64_t mid = (lo + hi) >> 1;
          if (offv(mid) <= c) lo = mid; else hi = mid;
        }
        const int64_t s0 = cuv(lo) + (c - offv(lo)) * kC;
        e = make_int2(static_cast<int>(s0),
                      static_cast<int>(min<int64_t>(kC, cuv(lo + 1) - s0)));
      }
      table[c] = e;
    }
  }
  if (!order) return;
  // Ranks are a permutation of [0, N): distinct (chunks, index) keys.
  for (int64_t n = tid; n < p.N; n += kT) {
    int64_t rank = n;
    if (small) {
      const int32_t cn = nchunks(n);
      rank = 0;
      for (int64_t m = 0; m < p.N; ++m) {
        const int32_t cm = nchunks(m);
        rank += (cm > cn) || (cm == cn && m < n);
      }
    }
    order[rank] = static_cast<int32_t>(n);
  }
}

// Global chunk c -> sequence n, first token s, length L (1..64); false if c
// is past the last chunk.
template <class P>
__device__ __forceinline__ bool locate_chunk(const P& p, int64_t c, int64_t& n, int64_t& s,
                                             int& L) {
  if (c >= p.chunk_off[p.N]) return false;
  int64_t lo = 0, hi = p.N;  // chunk_off[lo] <= c < chunk_off[hi]
  while (hi - lo > 1) {
    const int64_t mid = (lo + hi) >> 1;
    if (p.chunk_off[mid] <= c) lo = mid; else hi = mid;
  }
  n = lo;
  const int64_t ci = c - p.chunk_off[n];
  const int64_t a = cu_at(p, n), b = cu_at(p, n + 1);
  s = a + ci * kC;
  L = static_cast<int>(min<int64_t>(kC, b - s));
  return true;
}

// Up to kWaveSeqs sequences, a kernel finds its chunk or its sequence from
// cu_seqlens within each wave (lane m reads sequence m), and no offsets
// kernel runs before it: one round of loads at the start of every block
// instead of the dependent loads of a binary search over chunk_off, and one
// launch less per call.  Every lane of the wave must be active.
constexpr int64_t kWaveSeqs = 64;

// Inclusive wave64 prefix sum on DPP moves (no LDS round trips): shifts by
// 1, 2, 4, 8 within each 16-lane row (lanes shifted in from outside the row
// read 0), then row 0's total into row 1 and row 2's into row 3
// (row_bcast:15), then lane 31's running total into rows 2 and 3
// (row_bcast:31).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int32_t dpp_i32(int32_t v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, ROW_MASK, 0xF, true);
}
__device__ __forceinline__ int32_t wave_incl_scan(int32_t x) {
  x += dpp_i32<0x111>(x);       // row_shr:1
  x += dpp_i32<0x112>(x);       // row_shr:2
  x += dpp_i32<0x114>(x);       // row_shr:4
  x += dpp_i32<0x118>(x);       // row_shr:8
  x += dpp_i32<0x142, 0xA>(x);  // row_bcast:15 into rows 1, 3
  x += dpp_i32<0x143, 0xC>(x);  // row_bcast:31 into rows 2, 3
  return x;
}

struct WaveSeqs {
  int64_t a, b;  // sequence lane's first and end token (0, 0 past N)
  int32_t cnt;   // its chunks
  int32_t incl;  // chunks of sequences 0 .. lane (inclusive scan)
};
template <class P>
__device__ __forceinline__ WaveSeqs wave_seqs(const P& p) {
  const int lane = threadIdx.x & (kWave - 1);
  WaveSeqs w;
  const bool in = lane < p.N;
  w.a = in ? cu_at(p, lane) : 0;
  w.b = in ? cu_at(p, lane + 1) : 0;
  const int64_t len = w.b - w.a;
  w.cnt = static_cast<int32_t>(len > 0 ? (len + kC - 1) / kC : 0);
  w.incl = wave_incl_scan(w.cnt);
  return w;
}
__device__ __forceinline__ int64_t readlane64(int64_t v, int l) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), l);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32), l);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// locate_chunk for N <= kWaveSeqs (wave-uniform results).
template <class P>
__device__ __forceinline__ bool wave_locate_chunk(const P& p, int64_t c, int64_t& n, int64_t& s,
                                                  int& L) {
  const WaveSeqs w = wave_seqs(p);
  const int32_t total = __builtin_amdgcn_readlane(w.incl, kWave - 1);
  if (c >= total) return false;
  // Sequences that end at or before chunk c form a prefix of the lanes.
  const int nn = __popcll(__ballot(w.incl <= c));
  n = nn;
  const int32_t off = __builtin_amdgcn_readlane(w.incl - w.cnt, nn);
  s = readlane64(w.a, nn) + (c - off) * kC;
  L = static_cast<int>(min<int64_t>(kC, readlane64(w.b, nn) - s));
  return true;
}

// The sequence of rank r, longest first with ties by index (the order of
// chunk_offsets_kernel), and its first global chunk, for N <= kWaveSeqs.
template <class P>
__device__ __forceinline__ void wave_rank_seq(const P& p, int64_t r, int64_t& n, int64_t& c0) {
  const int lane = threadIdx.x & (kWave - 1);
  const WaveSeqs w = wave_seqs(p);
  int32_t rank = 0;
  for (int m = 0; m < static_cast<int>(p.N); ++m) {
    const int32_t cm = __builtin_amdgcn_readlane(w.cnt, m);
    rank += (cm > w.cnt) || (cm == w.cnt && m < lane);
  }
  const uint64_t hit = __ballot(lane < p.N && rank == r);
  const int nn = hit ? static_cast<int>(__builtin_ctzll(hit)) : 0;
  n = nn;
  c0 = __builtin_amdgcn_readlane(w.incl - w.cnt, nn);
}

// Chunk and sequence lookups that take the wave path when N allows and
// else read what chunk_offsets_kernel wrote.
template <class P>
__device__ __forceinline__ bool find_chunk(const P& p, int64_t c, int64_t& n, int64_t& s, int& L) {
  return p.N <= kWaveSeqs ? wave_locate_chunk(p, c, n, s, L) : locate_chunk(p, c, n, s, L);
}
template <class P>
__device__ __forceinline__ void find_ranked_seq(const P& p, int64_t r, int64_t& n, int64_t& c0) {
  if (p.N <= kWaveSeqs) {
    wave_rank_seq(p, r, n, c0);
  } else {
    n = p.seq_order[r];
    c0 = p.chunk_off[n];
  }
}

// 16x16x16 bf16 MFMA: lane l holds A[l%16][4(l/16)+e], B[4(l/16)+e][l%16]
// and C[4(l/16)+i][l%16], so a C fragment is already a B operand.
__device__ __forceinline__ f4_t mfma16k16(s4_t a, s4_t b, f4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ void split4s(const f4_t& x, s4_t& h, s4_t& l) {
  Vec<__bf16, 4> hh, ll;
  split4(x, hh, ll);
  h = __builtin_bit_cast(s4_t, hh);
  l = __builtin_bit_cast(s4_t, ll);
}
// hi/lo-split product (hi*hi + hi*lo + lo*hi) on 16x16x16 tiles.
__device__ __forceinline__ f4_t mfma16k16_split3(s4_t ah, s4_t al, s4_t bh, s4_t bl, f4_t c) {
  c = mfma16k16(ah, bh, c);
  c = mfma16k16(ah, bl, c);
  return mfma16k16(al, bh, c);
}

// ---------------------------------------------------------------------------
// X <- (I + M)^-1 for a strictly lower M in the wave's LDS tile X (only the
// strictly lower entries of the ten lower 16x16 tiles are read); the result
// is written back row-major (fp32, zeros above the diagonal).  One wave.
//   * the four 16x16 diagonal blocks by forward substitution, lane (g, c)
//     forming column c of X_gg: x[i] = delta_{i,c} - sum_{j<i} M[i][j] x[j];
//   * each pair of them merged into a 32x32 block, X_10 = -X_11 (M_10 X_00)
//     on 16x16x16 hi/lo-split MFMAs;
//   * the two 32x32 blocks merged the same way on 16x16x32 MFMAs.
// This is the 16->64 block merge of solve_tril.py:266-320.  Against 32x32
// diagonal blocks by substitution (a 32-deep chain of up to 31 FMAs per
// lane, 496 per lane in all; 120 now), measured on MI355X at config 4: the
// chunked prep kernel 83.1 -> 76.1 us, solve_tril 49.1 -> 40.8 us.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void invert_unit_lower(float (*X)[kLd]) {
  const int lane = threadIdx.x & 63;
  const int l15 = lane & 15, lg = lane >> 4;
  const int b = lane >> 5, cc = lane & 31;
  const f4_t zero = {0.f, 0.f, 0.f, 0.f};
  {
    // Diagonal blocks: group lg takes X_gg, g = lg.
    float x[16];
    const int o = 16 * lg;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float* mr = &X[o + i][o];
      float a0 = (i == l15) ? 1.f : 0.f, a1 = 0.f;
#pragma unroll
      for (int j = 0; j + 1 < i; j += 2) {
        a0 = fmaf(-mr[j], x[j], a0);
        a1 = fmaf(-mr[j + 1], x[j + 1], a1);
      }
      if (i & 1) a0 = fmaf(-mr[i - 1], x[i - 1], a0);
      x[i] = a0 + a1;
    }
    __builtin_amdgcn_wave_barrier();
    // Each group stores its block once transposed (a row of X_gg^T per
    // lane, 16-byte writes) and once row-major (a column per lane), at
    // disjoint places in spent diagonal blocks and the unused upper part:
    //   g = 0: X_0^T at [0,16)x[0,16)   (B operand below; part of X_00^T)
    //   g = 1: X_1^T at [16,32)x[16,32) (part of X_00^T), X_1 at [0,16)x[16,32)
    //   g = 2: X_2^T at [32,48)x[48,64) (B operand),      X_2 at [32,48)x[32,48)
    //   g = 3:                                            X_3 at [48,64)x[48,64)
    // and the unneeded two to [0,16)x[32,64), which the 64-merge rewrites.
    const int tr = (lg == 1 ? 16 : lg == 2 ? 32 : 0) + l15;
    const int tc = lg == 0 ? 0 : lg == 1 ? 16 : lg == 2 ? 48 : 32;
#pragma unroll
    for (int t = 0; t < 4; ++t)
      *reinterpret_cast<f4_t*>(&X[tr][tc + 4 * t]) = f4_t{x[4 * t], x[4 * t + 1], x[4 * t + 2], x[4 * t + 3]};
    const int cr = lg == 2 ? 32 : lg == 3 ? 48 : 0;
    const int ccol = (lg == 0 ? 48 : lg == 1 ? 16 : lg == 2 ? 32 : 48) + l15;
#pragma unroll
    for (int i = 0; i < 16; ++i) X[cr + i][ccol] = x[i];
  }
  __builtin_amdgcn_wave_barrier();
  // 16 -> 32: pair p (rows 32p ..): T = M' X_even, C = X_odd T, with M' =
  // M[32p+16 ..][32p ..], X_even from its transpose, X_odd row-major.
  f4_t cp[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    const int o = 32 * p;
    s4_t a1h, a1l, b1h, b1l, a2h, a2l, th, tl;
    split4s(*reinterpret_cast<const f4_t*>(&X[o + 16 + l15][o + 4 * lg]), a1h, a1l);
    split4s(*reinterpret_cast<const f4_t*>(&X[o + l15][o + 16 * p + 4 * lg]), b1h, b1l);
    const f4_t t = mfma16k16_split3(a1h, a1l, b1h, b1l, zero);
    split4s(t, th, tl);
    split4s(*reinterpret_cast<const f4_t*>(&X[p ? 48 + l15 : l15][16 + 32 * p + 4 * lg]), a2h, a2l);
    cp[p] = mfma16k16_split3(a2h, a2l, th, tl, zero);
  }
  __builtin_amdgcn_wave_barrier();
  // X_00 transposed into [0,32)^2: -C_0 transposed (16-byte writes) and the
  // zero block; X_11 row-major into [32,64)^2: -C_0's partner -C_1 and the
  // zero block.  Lane (lg, l15) holds C[4 lg + i][l15].
  *reinterpret_cast<f4_t*>(&X[l15][16 + 4 * lg]) = -cp[0];
  *reinterpret_cast<f4_t*>(&X[16 + l15][4 * lg]) = zero;
  *reinterpret_cast<f4_t*>(&X[32 + l15][48 + 4 * lg]) = zero;
#pragma unroll
  for (int i = 0; i < 4; ++i) X[48 + 4 * lg + i][32 + l15] = -cp[1][i];
  __builtin_amdgcn_wave_barrier();

  // T = M_10 X_00 (32 x 32).
  f4_t tt[2][2];
  {
    bf8_t bh[2], bl[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) split8(&X[nt * 16 + l15][8 * lg], bh[nt], bl[nt]);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      bf8_t ah, al;
      split8(&X[32 + mt * 16 + l15][8 * lg], ah, al);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        tt[mt][nt] = mfma_split3(ah, al, bh[nt], bl[nt], f4_t{0.f, 0.f, 0.f, 0.f});
    }
  }
  // T transposed into the unused upper-right block: X[n][32 + k] = T[k][n].
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
      *reinterpret_cast<f4_t*>(&X[nt * 16 + l15][32 + mt * 16 + 4 * lg]) = tt[mt][nt];
  __builtin_amdgcn_wave_barrier();
  // X_10 = -X_11 T.
  f4_t x10[2][2];
  {
    bf8_t bh[2], bl[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) split8(&X[nt * 16 + l15][32 + 8 * lg], bh[nt], bl[nt]);
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      bf8_t ah, al;
      split8(&X[32 + mt * 16 + l15][32 + 8 * lg], ah, al);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
        x10[mt][nt] = mfma_split3(ah, al, bh[nt], bl[nt], f4_t{0.f, 0.f, 0.f, 0.f});
    }
  }
  // Column cc of X_00 (lanes 0..31), read back from its transpose.
  float x[32];
  if (b == 0) {
#pragma unroll
    for (int i = 0; i < 32; i += 4) {
      const f4_t v = *reinterpret_cast<const f4_t*>(&X[cc][i]);
      x[i] = v[0];
      x[i + 1] = v[1];
      x[i + 2] = v[2];
      x[i + 3] = v[3];
    }
  }
  __builtin_amdgcn_wave_barrier();
  // Assemble row-major: X_10 over M_10, X_00 over its transpose, zeros over T.
#pragma unroll
  for (int mt = 0; mt < 2; ++mt)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int i = 0; i < 4; ++i) X[32 + mt * 16 + 4 * lg + i][nt * 16 + l15] = -x10[mt][nt][i];
  if (b == 0) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      X[i][cc] = x[i];
      X[i][32 + cc] = 0.f;
    }
  }
  __builtin_amdgcn_wave_barrier();
}

inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t{255}; }

}  // namespace gdn
}  // namespace xk
