// Row-normalisation kernels for gfx950: grouped LayerNorm / RMSNorm with an
// optional SiLU gate (layer_norm_fwd), Gemma RMSNorm and last-dim L2 norm.
//
// Semantics follow the reference's layer_norm_fwd
// (triton_npu/triton_src/test_layernorm_fwd.py:1120-1190 and the CPU golden
// triton_npu/test/triton_layernorm_fwd_test.cpp:37-116):
//   xg   = x * silu-gate(z)         if z given and !norm_before_gate
//   mean = sum(xg)/G, var = sum((xg-mean)^2)/G   (RMS: var = sum(xg^2)/G)
//   rstd = 1/sqrt(var + eps)
//   y    = (xg - mean) * rstd * w + b  (RMS: xg * rstd * w + b)
//   y   *= silu-gate(z)             if z given and norm_before_gate
//   mean/rstd stored at group * M + row.
//
// Design (HBM-bound, one read of x, one write of y):
//  * A "team" of TPG lanes owns one (row, group) item and holds the whole
//    group in registers as packed 16-byte vectors (NV per lane).  For the
//    common sizes (G <= 512 vectors) the team is at most one wave, so both
//    statistics are wave64 shuffle reductions with no LDS and no barrier.
//  * Blocks are persistent (as many as fit on the chip at once) and walk
//    items with a grid stride; x, z and y move with non-temporal 16-byte
//    accesses, weights with cached 16-byte loads (they are re-read by every
//    row and stay in L1/L2).
//  * Statistics: sum and sum of squares in one pass (gfx950 dot2 for 16-bit
//    inputs: exact products, fp32 accumulation, no unpacking), then
//    var = E[x^2] - mean^2; when mean^2 > 16 var a centred second pass over
//    the registers recomputes var exactly, so no digits are lost to
//    cancellation.
#include <type_traits>

#include "xk_common.h"

namespace xk {
namespace {

// Team-wide sum for TPG lanes (TPG <= 1024).  `red` is LDS scratch with one
// slot per wave of the block; only teams wider than a wave use it.
template <int TPG>
__device__ __forceinline__ float team_sum(float v, float* red) {
  if constexpr (TPG <= kWave) {
    return group_sum<TPG>(v);
  } else {
    v = group_sum<kWave>(v);
    constexpr int kWaves = TPG / kWave;
    const int wid = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    __syncthreads();  // previous readers of `red` are done
    if (lane == 0) red[wid] = v;
    __syncthreads();
    // Sum the waves of this team only (a block may hold several teams).
    const int base = (threadIdx.x / TPG) * kWaves;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) s += red[base + i];
    return s;
  }
}

// team_sum of two values at once: one exchange through `red` (two floats
// per wave) and two barriers instead of four.
template <int TPG>
__device__ __forceinline__ void team_sum2(float& a, float& b, float* red) {
  if constexpr (TPG <= kWave) {
    a = group_sum<TPG>(a);
    b = group_sum<TPG>(b);
  } else {
    a = group_sum<kWave>(a);
    b = group_sum<kWave>(b);
    constexpr int kWaves = TPG / kWave;
    const int wid = threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    __syncthreads();  // previous readers of `red` are done
    if (lane == 0) {
      red[2 * wid] = a;
      red[2 * wid + 1] = b;
    }
    __syncthreads();
    const int base = (threadIdx.x / TPG) * kWaves;
    float sa = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) {
      sa += red[2 * (base + i)];
      sb += red[2 * (base + i) + 1];
    }
    a = sa;
    b = sb;
  }
}

struct NormParams {
  const void* x;
  void* y;
  const void* w;
  const void* b;
  const void* z;
  float* mean;
  float* rstd;
  int64_t sx, sy, sz;  // row strides (elements)
  int64_t M, N, G;     // rows, row length, group size
  int64_t ngroups;
  float eps;
  float w_offset;  // 0 for layer_norm_fwd, 1 for Gemma (1 + gamma)
  int norm_before_gate;
  int is_rms;
  xk_dtype wdtype;
};

// Sum and sum of squares of one packed vector.  16-bit types use the
// gfx950 dot2 instructions (exact products, fp32 accumulation, one
// instruction per element pair and no unpacking); fp32 uses FMAs.
template <typename T, int VEC>
__device__ __forceinline__ void vec_sums(const Vec<T, VEC>& v, float& s1,
                                         float& s2) {
  if constexpr (std::is_same<T, bf16>::value) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    const bf2 one = {static_cast<bf16>(1.0f), static_cast<bf16>(1.0f)};
#pragma unroll
    for (int u = 0; u < VEC; u += 2) {
      const bf2 pr = {v.v[u], v.v[u + 1]};
      s1 = __builtin_amdgcn_fdot2_f32_bf16(pr, one, s1, false);
      s2 = __builtin_amdgcn_fdot2_f32_bf16(pr, pr, s2, false);
    }
  } else if constexpr (std::is_same<T, f16>::value) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 one = {static_cast<f16>(1.0f), static_cast<f16>(1.0f)};
#pragma unroll
    for (int u = 0; u < VEC; u += 2) {
      const h2 pr = {v.v[u], v.v[u + 1]};
      s1 = __builtin_amdgcn_fdot2(pr, one, s1, false);
      s2 = __builtin_amdgcn_fdot2(pr, pr, s2, false);
    }
  } else {
#pragma unroll
    for (int u = 0; u < VEC; ++u) {
      const float f = to_f32(v.v[u]);
      s1 += f;
      s2 = fmaf(f, f, s2);
    }
  }
}

// One (row, group) item per team.  FULL: the group is exactly
// NV * TPG * VEC elements, so no lane ever needs a bounds mask and all
// loads of an item issue back to back with no branch between them.
template <typename T, typename WT, int VEC, int TPG, int NV, bool HAS_Z,
          bool FULL>
__global__ void __launch_bounds__(TPG > 256 ? TPG : 256)
    ln_tile_kernel(NormParams p) {
  constexpr int kBlock = TPG > 256 ? TPG : 256;
  constexpr int kTeams = kBlock / TPG;
  constexpr bool kPair = VEC % 2 == 0;
  using VT = Vec<T, VEC>;
  using VW = Vec<WT, VEC>;
  __shared__ float red[2 * (kBlock / kWave)];

  const int team = threadIdx.x / TPG;
  const int lane = threadIdx.x % TPG;
  // Item indices fit in 32 bits (checked on the host).
  const uint32_t items = static_cast<uint32_t>(p.M * p.ngroups);
  const uint32_t ngroups = static_cast<uint32_t>(p.ngroups);
  const uint32_t G = static_cast<uint32_t>(p.G);
  const uint32_t stride = gridDim.x * kTeams;
  // Teams of a block run the same number of iterations so that block-wide
  // reductions (TPG > 64) see all lanes; surplus iterations are inactive.
  const uint32_t iters = (items + stride - 1) / stride;
  const bool has_b = p.b != nullptr;
  const bool gate_first = HAS_Z && !p.norm_before_gate;
  const bool gate_last = HAS_Z && p.norm_before_gate;
  const float inv_g = 1.0f / static_cast<float>(p.G);
  // Without a bias the bias loads read the weight (valid memory) and are
  // multiplied by zero, so the output loop has no branch.
  const float b_scale = has_b ? 1.f : 0.f;
  const WT* bsrc = reinterpret_cast<const WT*>(has_b ? p.b : p.w);

  bool in_group[NV];
#pragma unroll
  for (int j = 0; j < NV; ++j)
    in_group[j] = FULL || (j * TPG + lane) * VEC < static_cast<int>(G);

  // Weight/bias vectors of the lane, reloaded only when the group changes.
  // They are fetched together with x, before any store of the item: on
  // gfx9 a load issued after a store waits for that store (one vmcnt
  // counter), which would serialise the output loop.
  VW wv[NV], bv[NV];
  uint32_t cur_grp = 0xffffffffu;

  uint32_t item = blockIdx.x * kTeams + team;
  for (uint32_t it = 0; it < iters; ++it, item += stride) {
    const bool active = item < items;
    const uint32_t row = active ? (ngroups == 1 ? item : item / ngroups) : 0;
    const uint32_t grp = active ? item - row * ngroups : 0;
    const int64_t col0 = static_cast<int64_t>(grp) * G + lane * VEC;
    const T* xr = reinterpret_cast<const T*>(p.x) + row * p.sx + col0;
    const T* zr = reinterpret_cast<const T*>(p.z) + row * p.sz + col0;
    T* yr = reinterpret_cast<T*>(p.y) + row * p.sy + col0;

    VT xv[NV], zv[NV];
    if (active) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        if (FULL || in_group[j]) {
          xv[j] = ld_stream(reinterpret_cast<const VT*>(xr + j * TPG * VEC));
          if constexpr (HAS_Z)
            zv[j] = ld_stream(reinterpret_cast<const VT*>(zr + j * TPG * VEC));
        } else {
#pragma unroll
          for (int u = 0; u < VEC; ++u) xv[j].v[u] = from_f32<T>(0.f);
        }
      }
      if (grp != cur_grp) {
        const WT* wr = reinterpret_cast<const WT*>(p.w) + col0;
        const WT* br = bsrc + col0;
#pragma unroll
        for (int j = 0; j < NV; ++j)
          if (FULL || in_group[j]) {
            wv[j] = *reinterpret_cast<const VW*>(wr + j * TPG * VEC);
            bv[j] = *reinterpret_cast<const VW*>(br + j * TPG * VEC);
          }
        cur_grp = grp;
      }
    } else {
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int u = 0; u < VEC; ++u) xv[j].v[u] = from_f32<T>(0.f);
    }

    auto xin = [&](int j, int u) {
      float v = to_f32(xv[j].v[u]);
      if constexpr (HAS_Z) v *= gate_first ? silu(to_f32(zv[j].v[u])) : 1.f;
      return v;
    };

    // Statistics: one fused pass for sum and sum of squares (masked lanes
    // hold zeros), with an exact centred second pass when the mean is large
    // enough for the E[x^2] - mean^2 form to lose digits.
    float s1 = 0.f, s2 = 0.f;
    if (kPair && !HAS_Z) {
#pragma unroll
      for (int j = 0; j < NV; ++j) vec_sums<T, VEC>(xv[j], s1, s2);
    } else {
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
          const float f = (FULL || in_group[j]) ? xin(j, u) : 0.f;
          s1 += f;
          s2 = fmaf(f, f, s2);
        }
    }
    team_sum2<TPG>(s1, s2, red);
    const float mean = p.is_rms ? 0.f : s1 * inv_g;
    float var = fmaxf(s2 * inv_g - mean * mean, 0.f);
    if (!p.is_rms && mean * mean > 16.f * var) {
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < NV; ++j)
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
          const float d = (FULL || in_group[j]) ? xin(j, u) - mean : 0.f;
          ss = fmaf(d, d, ss);
        }
      var = team_sum<TPG>(ss, red) * inv_g;
    }
    const float rstd = 1.0f / sqrtf(var + p.eps);

    if (active && lane == 0) {
      const int64_t o = static_cast<int64_t>(grp) * p.M + row;
      if (p.mean && !p.is_rms) p.mean[o] = mean;
      if (p.rstd) p.rstd[o] = rstd;
    }

    if (active) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        if (!(FULL || in_group[j])) continue;
        VT out;
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
          float v = fmaf((xin(j, u) - mean) * rstd,
                         to_f32(wv[j].v[u]) + p.w_offset,
                         to_f32(bv[j].v[u]) * b_scale);
          if constexpr (HAS_Z) v *= gate_last ? silu(to_f32(zv[j].v[u])) : 1.f;
          out.v[u] = from_f32<T>(v);
        }
        st_stream(reinterpret_cast<VT*>(yr + j * TPG * VEC), out);
      }
    }
  }
}

// Groups longer than one register tile: one 1024-lane block per item
// streams the group three times (sum, centred sum of squares, output).
// Only reached for group sizes above 16K (fp32) / 32K (16-bit) elements or
// unaligned groups above 1024 elements.
template <typename T>
__global__ void __launch_bounds__(1024)
    ln_stream_kernel(NormParams p) {
  __shared__ float red[1024 / kWave];
  const int64_t item = blockIdx.x;
  const int64_t row = item / p.ngroups;
  const int64_t grp = item % p.ngroups;
  const int64_t col0 = grp * p.G;
  const T* xr = reinterpret_cast<const T*>(p.x) + row * p.sx + col0;
  const T* zr = p.z ? reinterpret_cast<const T*>(p.z) + row * p.sz + col0
                    : nullptr;
  T* yr = reinterpret_cast<T*>(p.y) + row * p.sy + col0;
  const bool gate_first = zr && !p.norm_before_gate;
  auto xin = [&](int64_t e) {
    float v = to_f32(xr[e]);
    if (gate_first) v *= silu(to_f32(zr[e]));
    return v;
  };
  const float inv_g = 1.0f / static_cast<float>(p.G);
  float mean = 0.f;
  if (!p.is_rms) {
    float s = 0.f;
    for (int64_t e = threadIdx.x; e < p.G; e += 1024) s += xin(e);
    mean = team_sum<1024>(s, red) * inv_g;
  }
  float ss = 0.f;
  for (int64_t e = threadIdx.x; e < p.G; e += 1024) {
    const float d = xin(e) - mean;
    ss += d * d;
  }
  const float rstd = 1.0f / sqrtf(team_sum<1024>(ss, red) * inv_g + p.eps);
  if (threadIdx.x == 0) {
    const int64_t o = grp * p.M + row;
    if (p.mean && !p.is_rms) p.mean[o] = mean;
    if (p.rstd) p.rstd[o] = rstd;
  }
  const bool gate_last = zr && p.norm_before_gate;
  for (int64_t e = threadIdx.x; e < p.G; e += 1024) {
    float v = (xin(e) - mean) * rstd *
              (load_as_f32(p.w, col0 + e, p.wdtype) + p.w_offset);
    if (p.b) v += load_as_f32(p.b, col0 + e, p.wdtype);
    if (gate_last) v *= silu(to_f32(zr[e]));
    yr[e] = from_f32<T>(v);
  }
}

template <typename T, typename WT, int VEC, int TPG, int NV, bool HAS_Z,
          bool FULL>
int launch_tile_z(const NormParams& p, hipStream_t s) {
  constexpr int kBlock = TPG > 256 ? TPG : 256;
  constexpr int kTeams = kBlock / TPG;
  auto kern = ln_tile_kernel<T, WT, VEC, TPG, NV, HAS_Z, FULL>;
  // Persistent grid: as many blocks as can be resident at once; teams then
  // stride over the items.
  static int resident[64] = {0};
  int dev = 0;
  (void)hipGetDevice(&dev);
  int& per_cu = resident[dev & 63];
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, kBlock, 0) !=
            hipSuccess ||
        n <= 0)
      n = 2;
    per_cu = n;
  }
  // Wide groups (teams of a wave or more): a persistent grid; more than ~3
  // resident 256-lane blocks per CU only adds DRAM page contention for this
  // streaming pattern.  Narrow groups (many small items): one pass, every
  // team one item, which keeps the most loads in flight (group 128 bf16
  // with a gate: 96 -> 71 us for 524288 rows on MI355X).
  const int64_t items = p.M * p.ngroups;
  const int64_t blocks_per_cu = std::min(per_cu, std::max(1, 768 / kBlock));
  const int64_t grid =
      TPG < kWave ? cdiv(items, kTeams)
                  : std::min<int64_t>(cdiv(items, kTeams),
                                      static_cast<int64_t>(num_cus()) * blocks_per_cu);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(kBlock), 0, s, p);
  return launch_status();
}

template <typename T, typename WT, int VEC, int TPG, int NV>
int launch_tile(const NormParams& p, hipStream_t s) {
  const bool full = p.G == static_cast<int64_t>(NV) * TPG * VEC;
  if (p.z)
    return full ? launch_tile_z<T, WT, VEC, TPG, NV, true, true>(p, s)
                : launch_tile_z<T, WT, VEC, TPG, NV, true, false>(p, s);
  return full ? launch_tile_z<T, WT, VEC, TPG, NV, false, true>(p, s)
              : launch_tile_z<T, WT, VEC, TPG, NV, false, false>(p, s);
}

template <typename T, typename WT>
int run_norm(const NormParams& p, hipStream_t s) {
  constexpr int kV = 16 / sizeof(T);
  const bool fits = p.M * p.ngroups < (int64_t{1} << 31);
  const bool vec_ok = p.G % kV == 0 && p.sx % kV == 0 && p.sy % kV == 0 &&
                      (!p.z || p.sz % kV == 0) && aligned(p.x, 16) &&
                      aligned(p.y, 16) && (!p.z || aligned(p.z, 16)) &&
                      aligned(p.w, kV * sizeof(WT)) &&
                      (!p.b || aligned(p.b, kV * sizeof(WT)));
  if (fits && vec_ok) {
    // Narrow groups: two vectors per lane (more bytes in flight per lane,
    // one shuffle step fewer than one vector per lane).
    const int64_t nvec = p.G / kV;
    if (nvec <= 8) return launch_tile<T, WT, kV, 4, 2>(p, s);
    if (nvec <= 16) return launch_tile<T, WT, kV, 8, 2>(p, s);
    if (nvec <= 32) return launch_tile<T, WT, kV, 16, 2>(p, s);
    if (nvec <= 64) return launch_tile<T, WT, kV, 32, 2>(p, s);
    if (nvec <= 128) return launch_tile<T, WT, kV, 64, 2>(p, s);
    if (nvec <= 256) return launch_tile<T, WT, kV, 64, 4>(p, s);
    if (nvec <= 512) return launch_tile<T, WT, kV, 128, 4>(p, s);
    if (nvec <= 1024) return launch_tile<T, WT, kV, 256, 4>(p, s);
    if (nvec <= 2048) return launch_tile<T, WT, kV, 512, 4>(p, s);
    if (nvec <= 4096) return launch_tile<T, WT, kV, 1024, 4>(p, s);
  } else if (fits) {
    if (p.G <= 64) return launch_tile<T, WT, 1, 64, 1>(p, s);
    if (p.G <= 256) return launch_tile<T, WT, 1, 64, 4>(p, s);
    if (p.G <= 1024) return launch_tile<T, WT, 1, 64, 16>(p, s);
  }
  hipLaunchKernelGGL((ln_stream_kernel<T>), dim3(p.M * p.ngroups),
                     dim3(1024), 0, s, p);
  return launch_status();
}

template <typename T>
int run_norm_w(const NormParams& p, xk_dtype xdt, hipStream_t s) {
  if (p.wdtype == xdt) return run_norm<T, T>(p, s);
  if (p.wdtype == XK_F32) return run_norm<T, float>(p, s);
  return XK_ERR_UNSUPPORTED;  // weights must match x or be fp32
}

int run_norm_dtype(const NormParams& p, xk_dtype dt, hipStream_t s) {
  switch (dt) {
    case XK_F32: return run_norm_w<float>(p, dt, s);
    case XK_BF16: return run_norm_w<bf16>(p, dt, s);
    case XK_F16: return run_norm_w<f16>(p, dt, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}

// ---------------------------------------------------------------------------
// L2 norm over the last dim.  Rows of aligned 16-byte vectors use the team
// kernel below; other rows use one wave per row, of any length.
// ---------------------------------------------------------------------------
template <typename T, typename TO, int VEC>
__global__ void __launch_bounds__(256)
    l2norm_kernel(const T* __restrict__ x, TO* __restrict__ y, int64_t rows,
                  int64_t cols, float eps) {
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const T* xr = x + row * cols;
  TO* yr = y + row * cols;
  float ss = 0.f;
  for (int64_t e = lane * VEC; e < cols; e += kWave * VEC) {
    float v[VEC];
    load_vec_f32<T, VEC>(xr + e, v);
#pragma unroll
    for (int u = 0; u < VEC; ++u) ss += v[u] * v[u];
  }
  const float r = 1.0f / sqrtf(group_sum<kWave>(ss) + eps);
  for (int64_t e = lane * VEC; e < cols; e += kWave * VEC) {
    float v[VEC];
    load_vec_f32<T, VEC>(xr + e, v);
#pragma unroll
    for (int u = 0; u < VEC; ++u) v[u] *= r;
    store_vec_f32<TO, VEC>(yr + e, v);
  }
}

// Rows of up to 256 16-byte vectors: a team of TPG lanes per row holds the
// row in registers (NV vectors per lane, one non-temporal read), reduces the
// sum of squares with shuffles inside the team and writes once.  Teams are
// at most a wave wide, so there is no LDS and no barrier; rows are
// team-uniform, so a team that exits never leaves a partner lane behind.
template <typename T, typename TO, int VEC, int TPG, int NV>
__global__ void __launch_bounds__(256)
    l2norm_team_kernel(const T* __restrict__ x, TO* __restrict__ y, int64_t rows,
                       int cols, float eps) {
  constexpr int kTeams = 256 / TPG;
  const int team = threadIdx.x / TPG;
  const int lane = threadIdx.x % TPG;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kTeams + team;
  if (row >= rows) return;
  using VT = Vec<T, VEC>;
  using VO = Vec<TO, VEC>;
  const T* xr = x + row * cols;
  TO* yr = y + row * cols;
  VT v[NV];
  float s1 = 0.f, ss = 0.f;
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * TPG + lane) * VEC;
    if (c < cols) {
      v[j] = ld_stream(reinterpret_cast<const VT*>(xr + c));
    } else {
#pragma unroll
      for (int u = 0; u < VEC; ++u) v[j].v[u] = from_f32<T>(0.f);
    }
    vec_sums<T, VEC>(v[j], s1, ss);
  }
  const float r = 1.0f / sqrtf(group_sum<TPG>(ss) + eps);
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int c = (j * TPG + lane) * VEC;
    if (c < cols) {
      VO o;
#pragma unroll
      for (int u = 0; u < VEC; ++u) o.v[u] = from_f32<TO>(to_f32(v[j].v[u]) * r);
      st_stream(reinterpret_cast<VO*>(yr + c), o);
    }
  }
}

template <typename T, typename TO, int TPG, int NV>
int launch_l2norm_team(const void* x, void* y, int64_t rows, int64_t cols, float eps,
                       hipStream_t s) {
  constexpr int kV = 16 / sizeof(T);
  hipLaunchKernelGGL((l2norm_team_kernel<T, TO, kV, TPG, NV>), dim3(cdiv(rows, 256 / TPG)),
                     dim3(256), 0, s, static_cast<const T*>(x), static_cast<TO*>(y), rows,
                     static_cast<int>(cols), eps);
  return launch_status();
}

template <typename T, typename TO>
int run_l2norm(const void* x, void* y, int64_t rows, int64_t cols, float eps,
               hipStream_t s) {
  constexpr int kV = 16 / sizeof(T);
  if (cols % kV == 0 && aligned(x, 16) && aligned(y, kV * sizeof(TO)) &&
      rows <= (int64_t{1} << 40)) {
    const int64_t nvec = cols / kV;
    if (nvec <= 8) return launch_l2norm_team<T, TO, 4, 2>(x, y, rows, cols, eps, s);
    if (nvec <= 16) return launch_l2norm_team<T, TO, 8, 2>(x, y, rows, cols, eps, s);
    if (nvec <= 32) return launch_l2norm_team<T, TO, 16, 2>(x, y, rows, cols, eps, s);
    if (nvec <= 64) return launch_l2norm_team<T, TO, 32, 2>(x, y, rows, cols, eps, s);
    if (nvec <= 128) return launch_l2norm_team<T, TO, 64, 2>(x, y, rows, cols, eps, s);
    if (nvec <= 256) return launch_l2norm_team<T, TO, 64, 4>(x, y, rows, cols, eps, s);
  }
  const dim3 grid(cdiv(rows, 4));
  const bool v4 = cols % 4 == 0 && aligned(x, 4 * sizeof(T)) &&
                  aligned(y, 4 * sizeof(TO));
  if (v4)
    hipLaunchKernelGGL((l2norm_kernel<T, TO, 4>), grid, dim3(256), 0, s,
                       static_cast<const T*>(x), static_cast<TO*>(y), rows,
                       cols, eps);
  else
    hipLaunchKernelGGL((l2norm_kernel<T, TO, 1>), grid, dim3(256), 0, s,
                       static_cast<const T*>(x), static_cast<TO*>(y), rows,
                       cols, eps);
  return launch_status();
}

template <typename T>
int run_l2norm_out(const void* x, void* y, int64_t rows, int64_t cols,
                   float eps, xk_dtype od, hipStream_t s) {
  switch (od) {
    case XK_F32: return run_l2norm<T, float>(x, y, rows, cols, eps, s);
    case XK_BF16: return run_l2norm<T, bf16>(x, y, rows, cols, eps, s);
    case XK_F16: return run_l2norm<T, f16>(x, y, rows, cols, eps, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}

}  // namespace
}  // namespace xk

using namespace xk;

extern "C" int xk_layer_norm_fwd(const void* x, int64_t stride_x_row, void* y,
                                 int64_t stride_y_row, const void* weight,
                                 const void* bias, const void* z,
                                 int64_t stride_z_row, float* mean, float* rstd,
                                 int64_t M, int64_t N, int64_t group_size,
                                 float eps, int norm_before_gate,
                                 int is_rms_norm, xk_dtype dtype,
                                 xk_dtype wdtype, void* stream) {
  if (M < 0 || N <= 0 || group_size <= 0 || N % group_size != 0)
    return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(wdtype))
    return XK_ERR_UNSUPPORTED;
  if (M == 0) return XK_OK;
  if (!x || !y || !weight) return XK_ERR_INVALID;
  NormParams p{};
  p.x = x;
  p.y = y;
  p.w = weight;
  p.b = bias;
  p.z = z;
  p.mean = mean;
  p.rstd = rstd;
  p.sx = stride_x_row;
  p.sy = stride_y_row;
  p.sz = stride_z_row;
  p.M = M;
  p.N = N;
  p.G = group_size;
  p.ngroups = N / group_size;
  p.eps = eps;
  p.w_offset = 0.f;
  p.norm_before_gate = norm_before_gate;
  p.is_rms = is_rms_norm;
  p.wdtype = wdtype;
  return run_norm_dtype(p, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int xk_gemma_rms_norm(const void* x, int64_t stride_x_row, void* y,
                                 int64_t stride_y_row, const void* gamma,
                                 float* rstd, int64_t M, int64_t N, float eps,
                                 xk_dtype dtype, xk_dtype wdtype,
                                 void* stream) {
  if (M < 0 || N <= 0) return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(wdtype))
    return XK_ERR_UNSUPPORTED;
  if (M == 0) return XK_OK;
  if (!x || !y || !gamma) return XK_ERR_INVALID;
  NormParams p{};
  p.x = x;
  p.y = y;
  p.w = gamma;
  p.rstd = rstd;
  p.sx = stride_x_row;
  p.sy = stride_y_row;
  p.M = M;
  p.N = N;
  p.G = N;
  p.ngroups = 1;
  p.eps = eps;
  p.w_offset = 1.f;
  p.norm_before_gate = 1;
  p.is_rms = 1;
  p.wdtype = wdtype;
  return run_norm_dtype(p, dtype, static_cast<hipStream_t>(stream));
}

extern "C" int xk_l2norm_last_dim(const void* x, void* y, int64_t rows,
                                  int64_t cols, float eps, xk_dtype dtype,
                                  xk_dtype out_dtype, void* stream) {
  if (rows < 0 || cols <= 0) return XK_ERR_INVALID;
  if (rows == 0) return XK_OK;
  if (!x || !y) return XK_ERR_INVALID;
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case XK_F32: return run_l2norm_out<float>(x, y, rows, cols, eps, out_dtype, s);
    case XK_BF16: return run_l2norm_out<bf16>(x, y, rows, cols, eps, out_dtype, s);
    case XK_F16: return run_l2norm_out<f16>(x, y, rows, cols, eps, out_dtype, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}
