// Depthwise causal conv1d for gfx950: single-step state update (decode)
// and varlen prefill with conv-state slots.
//
// Update (xllm::kernel::npu::npu_causal_conv1d_update) follows
// causal_conv1d_update_ref (triton_npu/triton_src/test_causal_conv1d_update.py:
// 1158-1210, no cache_seqlens): per channel
//   xs   = cat(state[0:S], x[0:T])                 (S = state_len >= W-1)
//   out_t = act(bias + sum_j w[j] * xs[S-W+1+t+j])
//   state <- xs[T:T+S]
// with the slot taken from conv_state_indices and pad_slot_id slots skipped
// (test_causal_conv1d_update.py:886-939).
//
// Varlen (npu_causal_conv1d_update_v2) follows the CPU golden
// causal_conv1d_update_ref_v2 (triton_npu/test/triton_causal_conv1d_update_v2
// _test.cpp:59-229) and, for speculative decoding, the kernel
// test_causal_conv1d_update_v2.py:16-249: per sequence s of
// query_start_loc, history = state[in_slot][:, off : off+W-1] (zeros if
// in_slot is out of range), out_t = act(bias + conv(cat(history, x_s))), and
// the final state rule
//   state_len_run = eff_state_len - (max_query_len - len)   (reference rule)
//   len >= state_len_run : state[out_slot][:, :run] = x_s[len-run:]
//   else                 : state[out_slot][:, :keep] = state[in_slot][:,
//                          off+shift : off+shift+keep], then x_s
// where eff_state_len = W-1 (+ max_query_len-1 with spec decoding),
// off = accepted-1 and shift = 1 with spec decoding, else off = 0 and
// shift = len.  A "prefill" rule (state_len_run = eff_state_len for every
// sequence, i.e. the last W-1 inputs) is offered for full-prefill callers.
//
// Design: channels are the vector dimension (16-byte accesses along the
// contiguous channel axis); each lane walks a tile of tokens with the W-1
// previous inputs in a register window, so every x element is read from
// HBM once (plus a W-1 token halo per tile, served from L2) and every output
// written once.  Sequence boundaries inside a tile restart the window from
// the sequence's state history.  Prefill is one launch: tile edges are
// moved so that every token whose window reaches into a sequence's state
// history lies in the tile of the sequence's first token, and the lane that
// reads that history (for its channels) writes the sequence's final state
// after its token loop.  An output slot that is also the sequence's input
// slot is thus overwritten only after it was read.  This needs tiles longer
// than the history (kTileT > W - 1, asserted below) and no sequence whose
// output slot is another sequence's input slot in the same call (the
// reference kernel has the same requirement; include/xk_ops.h states it).
#include "xk_common.h"

namespace xk {
namespace {

__device__ __forceinline__ float act(float v, int silu_on) {
  return silu_on ? silu(v) : v;
}

// ---------------------------------------------------------------------------
// Decode update, width 4 / state_len 3 / one token, contiguous layout:
// x, out [B, D]; state [lines, D, 3]; weight [D, 4].  One lane owns 8
// channels: 48 contiguous bytes of state (3 x 16 B), 16 B of x, 64 B of
// weights, and writes 16 B of output plus 48 B of state.  The x and weight
// loads are issued before the slot lookup, so their latency overlaps the
// dependent index -> state chain; x, out and the state move with
// non-temporal accesses (read once, written once).  Small blocks (one wave)
// spread the short-lived work evenly over the CUs.
// ---------------------------------------------------------------------------
constexpr int kW4Block = 64;

template <typename T, typename WT>
__global__ void __launch_bounds__(kW4Block)
    conv1d_update_w4_kernel(const T* __restrict__ x, T* __restrict__ out,
                            T* __restrict__ state, int64_t state_line_stride,
                            const WT* __restrict__ w, xk_dtype wdt,
                            const void* __restrict__ bias,
                            const int32_t* __restrict__ idx, int32_t pad,
                            int64_t lines, int64_t B, int64_t D, int silu_on) {
  constexpr int kC = 8;
  const int64_t b = blockIdx.y;
  const int64_t c0 = (static_cast<int64_t>(blockIdx.x) * kW4Block + threadIdx.x) * kC;
  if (c0 >= D) return;
  using V8 = Vec<T, kC>;
  const V8 xv = ld_stream(reinterpret_cast<const V8*>(x + b * D + c0));
  // The 8 channels' 4 taps are 32 contiguous weights.
  const Vec<WT, 32> wv = *reinterpret_cast<const Vec<WT, 32>*>(w + c0 * 4);
  const int64_t slot = idx ? idx[b] : b;
  if ((idx && slot == pad) || slot < 0 || slot >= lines) return;
  T* st = state + slot * state_line_stride + c0 * 3;
  // 24 state values (channel-major: s[c*3 + k]) as three 8-element vectors.
  Arr<T, 24> s;
  // A whole wave's 64 lanes cover 512 channels, whose states are 3 KB of
  // contiguous memory: it is moved as three 1 KB vector loads / stores, each
  // lane's 48 bytes gathered (and scattered back) through LDS.  Direct
  // 48-byte-per-lane accesses touched 24 cache lines per instruction instead
  // of 8 and took config 3b from 7.4 to 9.3 us on MI355X.  A partial last
  // wave (D % 512 != 0) keeps the direct accesses.
  __shared__ V8 sm[3 * kW4Block];
  const int lane = threadIdx.x;
  const bool full = (static_cast<int64_t>(blockIdx.x) + 1) * kW4Block * kC <= D;
  V8* sw = reinterpret_cast<V8*>(state + slot * state_line_stride +
                                 static_cast<int64_t>(blockIdx.x) * kW4Block * kC * 3);
  if (full) {
    const V8 a0 = ld_stream(sw + lane);
    const V8 a1 = ld_stream(sw + kW4Block + lane);
    const V8 a2 = ld_stream(sw + 2 * kW4Block + lane);
    sm[lane] = a0;
    sm[kW4Block + lane] = a1;
    sm[2 * kW4Block + lane] = a2;
    __syncthreads();
    *reinterpret_cast<V8*>(&s.v[0]) = sm[3 * lane];
    *reinterpret_cast<V8*>(&s.v[8]) = sm[3 * lane + 1];
    *reinterpret_cast<V8*>(&s.v[16]) = sm[3 * lane + 2];
  } else {
    *reinterpret_cast<V8*>(&s.v[0]) = ld_stream(reinterpret_cast<const V8*>(st));
    *reinterpret_cast<V8*>(&s.v[8]) = ld_stream(reinterpret_cast<const V8*>(st) + 1);
    *reinterpret_cast<V8*>(&s.v[16]) = ld_stream(reinterpret_cast<const V8*>(st) + 2);
  }
  V8 ov;
  Arr<T, 24> ns;
#pragma unroll
  for (int c = 0; c < kC; ++c) {
    const int64_t ch = c0 + c;
    const float s0 = to_f32(s.v[c * 3 + 0]);
    const float s1 = to_f32(s.v[c * 3 + 1]);
    const float s2 = to_f32(s.v[c * 3 + 2]);
    const float xc = to_f32(xv.v[c]);
    float acc = bias ? load_as_f32(bias, ch, wdt) : 0.f;
    acc = fmaf(s0, to_f32(wv.v[c * 4 + 0]), acc);
    acc = fmaf(s1, to_f32(wv.v[c * 4 + 1]), acc);
    acc = fmaf(s2, to_f32(wv.v[c * 4 + 2]), acc);
    acc = fmaf(xc, to_f32(wv.v[c * 4 + 3]), acc);
    ov.v[c] = from_f32<T>(act(acc, silu_on));
    ns.v[c * 3 + 0] = s.v[c * 3 + 1];
    ns.v[c * 3 + 1] = s.v[c * 3 + 2];
    ns.v[c * 3 + 2] = xv.v[c];
  }
  st_stream(reinterpret_cast<V8*>(out + b * D + c0), ov);
  if (full) {
    __syncthreads();
    sm[3 * lane] = *reinterpret_cast<const V8*>(&ns.v[0]);
    sm[3 * lane + 1] = *reinterpret_cast<const V8*>(&ns.v[8]);
    sm[3 * lane + 2] = *reinterpret_cast<const V8*>(&ns.v[16]);
    __syncthreads();
    st_stream(sw + lane, sm[lane]);
    st_stream(sw + kW4Block + lane, sm[kW4Block + lane]);
    st_stream(sw + 2 * kW4Block + lane, sm[2 * kW4Block + lane]);
  } else {
    st_stream(reinterpret_cast<V8*>(st), *reinterpret_cast<const V8*>(&ns.v[0]));
    st_stream(reinterpret_cast<V8*>(st) + 1, *reinterpret_cast<const V8*>(&ns.v[8]));
    st_stream(reinterpret_cast<V8*>(st) + 2, *reinterpret_cast<const V8*>(&ns.v[16]));
  }
}

// ---------------------------------------------------------------------------
// Decode update, any width / state_len / seqlen / strides: one lane per
// (batch, channel).  All outputs are computed from the old state first, then
// the state is shifted in ascending order (each new value comes from an
// equal or later index, so in-place shifting is safe).
// ---------------------------------------------------------------------------
struct UpdateParams {
  const void* x;
  int64_t sxb, sxd, sxt;
  void* out;
  int64_t sob, sod, sot;
  void* state;
  int64_t ssl, ssd, sss;
  const void* w;
  int64_t swd, sww;
  xk_dtype wdt;
  const void* bias;
  const int32_t* idx;
  int32_t pad;
  int64_t lines;
  int64_t B, D, T, W, S;
  int silu_on;
};

template <typename T>
__global__ void __launch_bounds__(256) conv1d_update_generic_kernel(UpdateParams p) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (gid >= p.B * p.D) return;
  const int64_t b = gid / p.D;
  const int64_t c = gid - b * p.D;
  const int64_t slot = p.idx ? p.idx[b] : b;
  if ((p.idx && slot == p.pad) || slot < 0 || slot >= p.lines) return;
  const T* x = reinterpret_cast<const T*>(p.x) + b * p.sxb + c * p.sxd;
  T* o = reinterpret_cast<T*>(p.out) + b * p.sob + c * p.sod;
  T* st = reinterpret_cast<T*>(p.state) + slot * p.ssl + c * p.ssd;
  auto val = [&](int64_t i) {  // element i of cat(state, x)
    return i < p.S ? to_f32(st[i * p.sss]) : to_f32(x[(i - p.S) * p.sxt]);
  };
  const float bias = p.bias ? load_as_f32(p.bias, c, p.wdt) : 0.f;
  for (int64_t t = 0; t < p.T; ++t) {
    float acc = bias;
    for (int64_t j = 0; j < p.W; ++j)
      acc = fmaf(val(p.S - p.W + 1 + t + j), load_as_f32(p.w, c * p.swd + j * p.sww, p.wdt), acc);
    o[t * p.sot] = from_f32<T>(act(acc, p.silu_on));
  }
  for (int64_t i = 0; i < p.S; ++i) {
    const int64_t src = p.T + i;
    const T v = src < p.S ? st[src * p.sss] : x[(src - p.S) * p.sxt];
    st[i * p.sss] = v;
  }
}

// ---------------------------------------------------------------------------
// Varlen prefill.
// ---------------------------------------------------------------------------
struct VarlenParams {
  const void* x;
  int64_t sx;  // token stride of x
  void* out;
  int64_t so;
  void* state;
  int64_t ssl, ssd, sss;  // state strides: line, channel, token
  int64_t lines;
  int64_t S;  // state_len (tokens held per channel)
  const void* w;
  int64_t swd, sww;
  xk_dtype wdt;
  const void* bias;
  const int32_t* qsl;  // [B + 1]
  int B;
  const int32_t* slots;  // NULL: slot = sequence index
  int64_t slot_stride;   // elements between rows of a 2-D slot table
  int slot_2d;
  const int32_t* init_idx;  // column of the input slot (2-D table)
  const int32_t* last_idx;  // column of the output slot (2-D table)
  const int32_t* accepted;  // spec decoding: accepted tokens per sequence
  int64_t D;
  int W;
  int64_t num_tokens;  // rows of x (>= qsl[B])
  int max_query_len;
  int eff_state_len;
  int state_rule;  // 0: reference rule, 1: prefill rule
  int silu_on;
  int32_t pad;
  int w_vec;  // weights are [D, W] contiguous, x's dtype, 16-byte aligned
  int64_t ncb, ntt;  // prefill grid: channel blocks x token tiles
};

__device__ __forceinline__ int64_t resolve_slot(const VarlenParams& p, int s,
                                                const int32_t* col) {
  if (!p.slots) return s;
  if (!p.slot_2d) return p.slots[s];
  const int c = col ? col[s] : 0;
  return p.slots[static_cast<int64_t>(s) * p.slot_stride + c];
}

// Index of the sequence holding token t (qsl non-decreasing).
__device__ __forceinline__ int find_seq(const int32_t* qsl, int B, int64_t t) {
  int lo = 0, hi = B;  // answer in [0, B)
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (qsl[mid] <= t) lo = mid; else hi = mid;
  }
  return lo;
}

// Tokens per lane per tile (16 measured best on MI355X for 8192 channels:
// longer tiles leave too few blocks, shorter ones repeat the prologue).
#ifndef XK_CONV_TILE_T
#define XK_CONV_TILE_T 16
#endif
constexpr int kTileT = XK_CONV_TILE_T;
// Widths up to 8 (the entry point's limit) leave a history of up to 7
// inputs; the one-launch state write needs every tile to be longer than
// that (see tile_edge in the kernel).
static_assert(kTileT >= 8, "conv1d prefill tiles must be longer than the conv history");
#ifndef XK_CONV_GROUP
#define XK_CONV_GROUP 8
#endif
constexpr int kGroup = XK_CONV_GROUP;  // tokens loaded / computed together
// Prefetch the next group of tokens while computing the current one (no
// measurable gain at 32-token tiles; costs registers).
#ifndef XK_CONV_DBUF
#define XK_CONV_DBUF 0
#endif
constexpr bool kDoubleBuffer = XK_CONV_DBUF != 0;
// Non-temporal hints for the streamed x loads / output stores (bit 0:
// stores, bit 1: loads).
#ifndef XK_CONV_NT
#define XK_CONV_NT 3
#endif
constexpr bool kNtStore = (XK_CONV_NT & 1) != 0;
constexpr bool kNtLoad = (XK_CONV_NT & 2) != 0;

template <typename T, int W, int VEC, bool SILU>
__global__ void __launch_bounds__(256) conv1d_varlen_kernel(VarlenParams p) {
  using VT = Vec<T, VEC>;
  // XCD-aware block order: block b runs on XCD b % 8, and the remapped index
  // gives each XCD a contiguous run of (channel block, token tile) pairs,
  // token tiles fastest.  A tile's halo (the last W-1 inputs of the previous
  // tile) is then usually still in that XCD's L2.  The grid is 8 * per
  // blocks, so the remap is a permutation of [0, 8 * per).
  const int64_t nblk = p.ncb * p.ntt;
  const int64_t per = (nblk + 7) / 8;
  const int64_t bid = static_cast<int64_t>(blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (bid >= nblk) return;
  const int64_t tile = bid % p.ntt;
  const int64_t cb = bid / p.ntt;
  const int64_t c0 = (cb * 256 + threadIdx.x) * VEC;
  if (c0 >= p.D) return;
  // Tile k covers tokens [tile_edge(k * kTileT), tile_edge((k + 1) * kTileT)):
  // an edge that falls inside the first W-1 tokens of a sequence moves to the
  // end of those tokens.  Every token whose window reaches into the conv
  // state's history then sits in the tile of its sequence's first token, so
  // exactly one lane per (sequence, channel group) reads that history -- and
  // writes the sequence's final state right after reading it (below).  W-1
  // <= 7 < kTileT, so every tile keeps at least kTileT - 6 tokens.
  // The sequence holding token t, searched forward from sequence q (with
  // qsl[q] <= t or q = 0): a few steps cover the usual case (the next
  // sequence at most), a binary search the rest.  One search per block.
  auto seq_from = [&](int q, int64_t t) {
    for (int i = 0; i < 4; ++i) {
      if (q + 1 >= p.B || p.qsl[q + 1] > t) return q;
      ++q;
    }
    return find_seq(p.qsl, p.B, t);
  };
  // Edge b moved out of the first W-1 tokens of its sequence q.
  auto tile_edge = [&](int q, int64_t b) -> int64_t {
    if constexpr (W <= 2) {
      return b;  // the history reaches only the first token of a sequence
    } else {
      const int64_t st = p.qsl[q], en = p.qsl[q + 1];
      return (b > st && b < st + (W - 1) && b < en) ? min(st + (W - 1), en) : b;
    }
  };
  const int64_t e0 = tile * kTileT, e1 = e0 + kTileT;
  const int s_e0 = find_seq(p.qsl, p.B, e0);
  // Tokens outside [qsl[0], qsl[B]) belong to no sequence and are skipped.
  const int64_t t0 = max(tile_edge(s_e0, e0), static_cast<int64_t>(p.qsl[0]));
  const int64_t total = p.qsl[p.B];
  const int64_t t_end = min(min(tile_edge(seq_from(s_e0, e1), e1), total), p.num_tokens);
  if (t0 >= t_end) return;

  float wt[W][VEC], bs[VEC];
  constexpr int kWVec = 16 / sizeof(T);
  if constexpr ((VEC * W) % kWVec == 0) {
    if (p.w_vec) {
      // Weights [D, W] in x's dtype: the lane's VEC*W taps are contiguous
      // and 16-byte aligned, fetched as whole vectors.
      const T* wp = reinterpret_cast<const T*>(p.w) + c0 * W;
#pragma unroll
      for (int q = 0; q < VEC * W / kWVec; ++q) {
        const Vec<T, kWVec> wv = reinterpret_cast<const Vec<T, kWVec>*>(wp)[q];
#pragma unroll
        for (int e = 0; e < kWVec; ++e) {
          const int i = q * kWVec + e;
          wt[i % W][i / W] = to_f32(wv.v[e]);
        }
      }
    }
  }
  if (!p.w_vec || (VEC * W) % kWVec != 0) {
#pragma unroll
    for (int u = 0; u < VEC; ++u)
#pragma unroll
      for (int j = 0; j < W; ++j)
        wt[j][u] = load_as_f32(p.w, (c0 + u) * p.swd + j * p.sww, p.wdt);
  }
#pragma unroll
  for (int u = 0; u < VEC; ++u)
    bs[u] = p.bias ? load_as_f32(p.bias, c0 + u, p.wdt) : 0.f;

  int s = seq_from(s_e0, t0);
  int64_t seq_start = p.qsl[s];
  int64_t seq_end = p.qsl[s + 1];
  float win[W > 1 ? W - 1 : 1][VEC];
  bool skip = false;

  // Final conv state of sequence sq for this lane's channels, written after
  // the token loop by the lane that read the sequence's history (so an
  // output slot that is also the input slot is overwritten only after its
  // history was read).  The state_len_run rule of
  // triton_causal_conv1d_update_v2_test.cpp:138-223 (state_rule 0), or the
  // last eff inputs (state_rule 1); with speculative decoding the kept part
  // starts one column after the accepted token's window
  // (test_causal_conv1d_update_v2.py:326-333).
  auto write_state = [&](int sq) {
    const int64_t start = p.qsl[sq], len = p.qsl[sq + 1] - start;
    if (len <= 0 || start < 0 || start + len > p.num_tokens) return;
    const int64_t in_slot = resolve_slot(p, sq, p.init_idx);
    if (p.slots && in_slot == p.pad) return;
    const int s = sq;
    const int64_t out_slot = resolve_slot(p, s, p.last_idx);
    if (out_slot < 0 || out_slot >= p.lines) return;
    const bool in_valid = in_slot >= 0 && in_slot < p.lines;
    const int64_t run = p.state_rule == 0
                            ? p.eff_state_len - (p.max_query_len - len)
                            : p.eff_state_len;
    if (run <= 0 || run > p.S) return;
    const int64_t off = p.accepted ? p.accepted[s] - 1 : 0;
    const int64_t shift = p.accepted ? 1 : len;
#pragma unroll
    for (int u = 0; u < VEC; ++u) {
      const int64_t c = c0 + u;
      T* dst = reinterpret_cast<T*>(p.state) + out_slot * p.ssl + c * p.ssd;
      const T* src = reinterpret_cast<const T*>(p.state) + in_slot * p.ssl + c * p.ssd;
      const T* xs = reinterpret_cast<const T*>(p.x) + start * p.sx + c;
      if (len >= run) {
        for (int64_t i = 0; i < run; ++i) dst[i * p.sss] = xs[(len - run + i) * p.sx];
      } else {
        const int64_t keep = run - len;
        if (in_valid && off >= 0)
          for (int64_t i = 0; i < keep && off + shift + i < p.S; ++i)
            dst[i * p.sss] = src[(off + shift + i) * p.sss];  // reads run ahead of writes
        for (int64_t i = 0; i < len; ++i) dst[(keep + i) * p.sss] = xs[i * p.sx];
      }
    }
  };

  // Loads the state history of sequence s and, for a tile starting inside
  // the sequence, the preceding inputs, into the window.
  auto enter = [&](int64_t t) {
    const int64_t in_slot = resolve_slot(p, s, p.init_idx);
    skip = p.slots && in_slot == p.pad;
    const int64_t off = p.accepted ? p.accepted[s] - 1 : 0;
    // History entries must lie inside a real slot and its state_len.
    const bool valid = in_slot >= 0 && in_slot < p.lines && off >= 0 &&
                       off + (W - 1) <= p.S;
    const T* st = reinterpret_cast<const T*>(p.state) + in_slot * p.ssl + c0 * p.ssd;
#pragma unroll
    for (int j = 0; j < W - 1; ++j) {
      const int64_t pos = t - (W - 1) + j;  // token this window entry holds
      const int64_t v = (W - 1) + (pos - seq_start);  // index in cat(hist, x)
      if (v >= W - 1) {  // an earlier input of this sequence: one vector load
        const VT hv = *reinterpret_cast<const VT*>(
            reinterpret_cast<const T*>(p.x) + pos * p.sx + c0);
#pragma unroll
        for (int u = 0; u < VEC; ++u) win[j][u] = to_f32(hv.v[u]);
      } else {
#pragma unroll
        for (int u = 0; u < VEC; ++u)
          win[j][u] = (valid && !skip) ? to_f32(st[u * p.ssd + (off + v) * p.sss]) : 0.f;
      }
    }
  };
  const int s_first = s;
  enter(t0);

  // One token through the window: returns the output vector.
  auto step = [&](const VT& xv) {
    VT ov;
#pragma unroll
    for (int u = 0; u < VEC; ++u) {
      const float xc = to_f32(xv.v[u]);
      float acc = bs[u];
#pragma unroll
      for (int j = 0; j < W - 1; ++j) acc = fmaf(win[j][u], wt[j][u], acc);
      acc = fmaf(xc, wt[W - 1][u], acc);
      if constexpr (SILU) acc = silu(acc);
      ov.v[u] = from_f32<T>(acc);
#pragma unroll
      for (int j = 0; j + 1 < W - 1; ++j) win[j][u] = win[j + 1][u];
      if constexpr (W > 1) win[W - 2][u] = xc;
    }
    return ov;
  };

  const T* xp = reinterpret_cast<const T*>(p.x) + t0 * p.sx + c0;
  T* op = reinterpret_cast<T*>(p.out) + t0 * p.so + c0;
  int64_t t = t0;
  while (t < t_end) {
    if (t + kGroup <= seq_end && t + kGroup <= t_end) {
      // Fast path: runs of kGroup tokens inside one sequence, straight-line
      // code.  The next group's loads are issued before the current group
      // is computed (two register sets), so a lane overlaps its own loads
      // with its arithmetic.
      VT xs[kGroup];
#pragma unroll
      for (int k = 0; k < kGroup; ++k)
        xs[k] = kNtLoad ? ld_stream(reinterpret_cast<const VT*>(xp + k * p.sx))
                        : *reinterpret_cast<const VT*>(xp + k * p.sx);
      while (true) {
        const bool more = kDoubleBuffer && t + 2 * kGroup <= seq_end &&
                          t + 2 * kGroup <= t_end;
        VT nx[kGroup];
        if (more) {
#pragma unroll
          for (int k = 0; k < kGroup; ++k)
            nx[k] = *reinterpret_cast<const VT*>(xp + (kGroup + k) * p.sx);
        }
#pragma unroll
        for (int k = 0; k < kGroup; ++k) {
          const VT ov = step(xs[k]);
          if (!skip) {
            if (kNtStore) st_stream(reinterpret_cast<VT*>(op + k * p.so), ov);
            else *reinterpret_cast<VT*>(op + k * p.so) = ov;
          }
        }
        t += kGroup;
        xp += kGroup * p.sx;
        op += kGroup * p.so;
        if (!more) break;
#pragma unroll
        for (int k = 0; k < kGroup; ++k) xs[k] = nx[k];
      }
      continue;
    }
    // Slow path: one token, crossing into the next non-empty sequence when
    // needed (its window is then pure history).
    if (t >= seq_end) {
      do {
        ++s;
        seq_start = p.qsl[s];
        seq_end = p.qsl[s + 1];
      } while (t >= seq_end);
      enter(t);
    }
    const VT ov = step(*reinterpret_cast<const VT*>(xp));
    if (!skip) *reinterpret_cast<VT*>(op) = ov;
    ++t;
    xp += p.sx;
    op += p.so;
  }
  // Final states of the sequences whose first token lies in this tile:
  // their histories were all read above, by this lane.
  for (int sq = s_first; sq < p.B && p.qsl[sq] < t_end; ++sq)
    if (p.qsl[sq] >= t0) write_state(sq);
}

template <typename T, int VEC>
int launch_varlen_w(VarlenParams p, hipStream_t s) {
  p.ncb = cdiv(p.D, 256 * VEC);
  p.ntt = cdiv(p.num_tokens, kTileT);
  const int64_t per = cdiv(p.ncb * p.ntt, 8);
  if (8 * per > INT32_MAX) return XK_ERR_UNSUPPORTED;
  const dim3 grid(static_cast<uint32_t>(8 * per));
  switch (p.W) {
#define XK_W(n) \
  case n:                                                                       \
    if (p.silu_on)                                                              \
      hipLaunchKernelGGL((conv1d_varlen_kernel<T, n, VEC, true>), grid, dim3(256), 0, s, p); \
    else                                                                        \
      hipLaunchKernelGGL((conv1d_varlen_kernel<T, n, VEC, false>), grid, dim3(256), 0, s, p); \
    break;
    XK_W(1) XK_W(2) XK_W(3) XK_W(4) XK_W(5) XK_W(6) XK_W(7) XK_W(8)
#undef XK_W
    default: return XK_ERR_UNSUPPORTED;
  }
  return launch_status();
}

template <typename T>
int launch_varlen(VarlenParams p, xk_dtype dt, hipStream_t s) {
  constexpr int kV = 16 / sizeof(T);
  const bool vec = p.D % kV == 0 && p.sx % kV == 0 && p.so % kV == 0 &&
                   aligned(p.x, 16) && aligned(p.out, 16);
  p.w_vec = p.wdt == dt && p.swd == p.W && p.sww == 1 && aligned(p.w, 16);
  return vec ? launch_varlen_w<T, kV>(p, s) : launch_varlen_w<T, 1>(p, s);
}

}  // namespace
}  // namespace xk

using namespace xk;

extern "C" int xk_causal_conv1d_update(
    const void* x, int64_t stride_x_batch, int64_t stride_x_dim,
    int64_t stride_x_token, void* conv_state, int64_t stride_state_line,
    int64_t stride_state_dim, int64_t stride_state_token,
    const void* weight, int64_t stride_w_dim, int64_t stride_w_tap,
    const void* bias, xk_dtype wdtype, const int32_t* conv_state_indices,
    int32_t pad_slot_id, int64_t num_cache_lines, void* out,
    int64_t stride_o_batch,
    int64_t stride_o_dim, int64_t stride_o_token, int64_t batch, int64_t dim,
    int64_t seqlen, int64_t width, int64_t state_len, int activation,
    xk_dtype dtype, void* stream) {
  if (batch < 0 || dim <= 0 || seqlen <= 0 || width <= 0 ||
      state_len < width - 1)
    return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(wdtype)) return XK_ERR_UNSUPPORTED;
  if (batch == 0) return XK_OK;
  if (!x || !conv_state || !weight || !out) return XK_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int eb = elem_bytes(dtype);
  const bool w_ok = (wdtype == dtype && aligned(weight, 64)) ||
                    (wdtype == XK_F32 && aligned(weight, 128));
  const bool fast = width == 4 && state_len == 3 && seqlen == 1 &&
                    stride_x_dim == 1 && stride_o_dim == 1 &&
                    stride_state_dim == 3 && stride_state_token == 1 &&
                    stride_w_dim == 4 && stride_w_tap == 1 && eb == 2 && w_ok &&
                    dim % 8 == 0 && stride_x_batch == dim &&
                    stride_o_batch == dim && stride_state_line % 8 == 0 &&
                    aligned(x, 16) && aligned(out, 16) && aligned(conv_state, 16);
  if (fast) {
    const dim3 grid(cdiv(dim, kW4Block * 8), batch);
#define XK_W4(T, WT)                                                            \
  hipLaunchKernelGGL((conv1d_update_w4_kernel<T, WT>), grid, dim3(kW4Block), 0, s, \
                     static_cast<const T*>(x), static_cast<T*>(out),            \
                     static_cast<T*>(conv_state), stride_state_line,            \
                     static_cast<const WT*>(weight), wdtype, bias,              \
                     conv_state_indices, pad_slot_id, num_cache_lines, batch,   \
                     dim, activation)
    if (dtype == XK_BF16) {
      if (wdtype == XK_F32) XK_W4(bf16, float); else XK_W4(bf16, bf16);
    } else {
      if (wdtype == XK_F32) XK_W4(f16, float); else XK_W4(f16, f16);
    }
#undef XK_W4
    return launch_status();
  }
  UpdateParams p{};
  p.x = x;
  p.sxb = stride_x_batch;
  p.sxd = stride_x_dim;
  p.sxt = stride_x_token;
  p.out = out;
  p.sob = stride_o_batch;
  p.sod = stride_o_dim;
  p.sot = stride_o_token;
  p.state = conv_state;
  p.ssl = stride_state_line;
  p.ssd = stride_state_dim;
  p.sss = stride_state_token;
  p.w = weight;
  p.swd = stride_w_dim;
  p.sww = stride_w_tap;
  p.wdt = wdtype;
  p.bias = bias;
  p.idx = conv_state_indices;
  p.pad = pad_slot_id;
  p.lines = num_cache_lines;
  p.B = batch;
  p.D = dim;
  p.T = seqlen;
  p.W = width;
  p.S = state_len;
  p.silu_on = activation;
  const dim3 grid(cdiv(batch * dim, 256));
  switch (dtype) {
    case XK_F32: hipLaunchKernelGGL(conv1d_update_generic_kernel<float>, grid, dim3(256), 0, s, p); break;
    case XK_BF16: hipLaunchKernelGGL(conv1d_update_generic_kernel<bf16>, grid, dim3(256), 0, s, p); break;
    default: hipLaunchKernelGGL(conv1d_update_generic_kernel<f16>, grid, dim3(256), 0, s, p); break;
  }
  return launch_status();
}

extern "C" int xk_causal_conv1d_varlen(
    const void* x, int64_t stride_x_token, int64_t num_tokens, void* out,
    int64_t stride_o_token, void* conv_state, int64_t stride_state_line,
    int64_t stride_state_dim, int64_t stride_state_token,
    int64_t num_cache_lines, int64_t state_len, const void* weight,
    int64_t stride_w_dim, int64_t stride_w_tap, const void* bias,
    xk_dtype wdtype, const int32_t* query_start_loc, int64_t batch,
    const int32_t* slot_table, int64_t slot_table_stride, int slot_table_2d,
    const int32_t* initial_state_idx, const int32_t* last_state_idx,
    const int32_t* num_accepted_tokens, int64_t dim, int64_t width,
    int64_t max_query_len, int state_rule, int activation,
    int32_t pad_slot_id, xk_dtype dtype, void* stream) {
  if (batch < 0 || dim <= 0 || width < 1 || width > 8 || num_tokens < 0 ||
      (state_rule != 0 && state_rule != 1) || max_query_len < 0)
    return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(wdtype)) return XK_ERR_UNSUPPORTED;
  const int64_t eff = width - 1 + (num_accepted_tokens ? max_query_len - 1 : 0);
  if (eff > state_len) return XK_ERR_INVALID;  // state cannot hold the history
  if (batch == 0 || num_tokens == 0) return XK_OK;
  if (!x || !out || !conv_state || !weight || !query_start_loc)
    return XK_ERR_INVALID;
  VarlenParams p{};
  p.x = x;
  p.sx = stride_x_token;
  p.out = out;
  p.so = stride_o_token;
  p.state = conv_state;
  p.ssl = stride_state_line;
  p.ssd = stride_state_dim;
  p.sss = stride_state_token;
  p.lines = num_cache_lines;
  p.S = state_len;
  p.w = weight;
  p.swd = stride_w_dim;
  p.sww = stride_w_tap;
  p.wdt = wdtype;
  p.bias = bias;
  p.qsl = query_start_loc;
  p.B = static_cast<int>(batch);
  p.slots = slot_table;
  p.slot_stride = slot_table_stride;
  p.slot_2d = slot_table_2d;
  p.init_idx = initial_state_idx;
  p.last_idx = last_state_idx;
  p.accepted = num_accepted_tokens;
  p.D = dim;
  p.W = static_cast<int>(width);
  p.num_tokens = num_tokens;
  p.max_query_len = static_cast<int>(max_query_len);
  p.eff_state_len = static_cast<int>(eff);
  p.state_rule = state_rule;
  p.silu_on = activation;
  p.pad = pad_slot_id;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case XK_F32: return launch_varlen<float>(p, dtype, s);
    case XK_BF16: return launch_varlen<bf16>(p, dtype, s);
    default: return launch_varlen<f16>(p, dtype, s);
  }
}
