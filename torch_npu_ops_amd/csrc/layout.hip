// Split of the GDN input projection into the conv1d input and the gates,
// for gfx950 (xllm::kernel::npu::npu_fused_qkvzba_split_reshape_cat).
//
// Semantics follow fused_qkvzba_split_reshape_cat_ref
// (triton_npu/triton_src/test_fused_qkvzba_split_reshape.py:463-506): with
// R = num_heads_v / num_heads_qk v heads per qk head, each row of
// mixed_qkvz holds num_heads_qk groups [q (hk) | k (hk) | v (R*hv) |
// z (R*hv)] and each row of mixed_ba holds groups [b (R) | a (R)].  The
// outputs are
//   mixed_qkv = [q of all groups | k of all groups | v of all groups]
//   z = [z of all groups] (v-head order), b and a likewise [num_heads_v].
// It is a pure permutation: every element is copied, bit for bit.
//
// Design (HBM-bound copy): one lane per 16-byte vector of the source row
// (head dims are multiples of the vector, so a vector never straddles two
// segments); reads are fully coalesced and each segment is written as a
// contiguous run.  The few b/a elements of a row are moved by the lanes past
// the row's last vector.  Blocks walk (row, chunk of the row) in a 1-D grid,
// so any number of rows fits.
#include "xk_common.h"

namespace xk {
namespace {

struct SplitParams {
  const void* qkvz;
  int64_t sq;  // row stride of mixed_qkvz (elements)
  const void* ba;
  int64_t sba;
  void* qkv;
  void* z;
  void* b;
  void* a;
  int64_t rows;
  int nqk, nv, hk, hv, R;
  int dt;      // group width in mixed_qkvz: 2 hk + 2 R hv
  int items;   // per row: vectors (or elements) of mixed_qkvz, then 2 nv gates
  int vec;     // elements per item of mixed_qkvz (1 or VEC)
  int64_t blocks_per_row;
};

template <typename T, typename TB, int VEC>
__global__ void __launch_bounds__(256) qkvzba_split_kernel(SplitParams p) {
  const int64_t blk = blockIdx.x;
  const int64_t row = blk / p.blocks_per_row;
  const int item = static_cast<int>((blk - row * p.blocks_per_row) * 256 + threadIdx.x);
  if (row >= p.rows || item >= p.items) return;
  const int nsrc = p.nqk * p.dt / VEC;  // source items of the qkvz row
  if (item < nsrc) {
    const int s = item * VEC;  // element offset in the row
    const int g = s / p.dt;
    const int r = s - g * p.dt;
    const int vd = p.R * p.hv;
    T* dst;
    if (r < 2 * p.hk) {  // q or k
      const int kpart = r >= p.hk;
      dst = reinterpret_cast<T*>(p.qkv) + row * (2 * p.nqk * p.hk + p.nv * p.hv) +
            kpart * p.nqk * p.hk + g * p.hk + (r - kpart * p.hk);
    } else if (r < 2 * p.hk + vd) {  // v
      dst = reinterpret_cast<T*>(p.qkv) + row * (2 * p.nqk * p.hk + p.nv * p.hv) +
            2 * p.nqk * p.hk + g * vd + (r - 2 * p.hk);
    } else {  // z
      dst = reinterpret_cast<T*>(p.z) + row * (p.nv * p.hv) + g * vd + (r - 2 * p.hk - vd);
    }
    using VT = Vec<T, VEC>;
    const T* src = reinterpret_cast<const T*>(p.qkvz) + row * p.sq + s;
    st_stream(reinterpret_cast<VT*>(dst), ld_stream(reinterpret_cast<const VT*>(src)));
  } else {
    const int e = item - nsrc;  // element of the ba row: group e / 2R
    const int g = e / (2 * p.R);
    const int j = e - g * 2 * p.R;
    const TB v = reinterpret_cast<const TB*>(p.ba)[row * p.sba + e];
    if (j < p.R)
      reinterpret_cast<TB*>(p.b)[row * p.nv + g * p.R + j] = v;
    else
      reinterpret_cast<TB*>(p.a)[row * p.nv + g * p.R + (j - p.R)] = v;
  }
}

template <typename T, typename TB>
int launch_split(SplitParams p, hipStream_t s) {
  constexpr int kV = 16 / sizeof(T);
  const bool vec = p.hk % kV == 0 && p.hv % kV == 0 && p.sq % kV == 0 &&
                   aligned(p.qkvz, 16) && aligned(p.qkv, 16) && aligned(p.z, 16);
  p.vec = vec ? kV : 1;
  p.items = p.nqk * p.dt / p.vec + 2 * p.nv;
  p.blocks_per_row = cdiv(p.items, 256);
  const int64_t blocks = p.rows * p.blocks_per_row;
  if (blocks > INT32_MAX) return XK_ERR_UNSUPPORTED;
  if (vec)
    hipLaunchKernelGGL((qkvzba_split_kernel<T, TB, kV>), dim3(static_cast<uint32_t>(blocks)),
                       dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((qkvzba_split_kernel<T, TB, 1>), dim3(static_cast<uint32_t>(blocks)),
                       dim3(256), 0, s, p);
  return launch_status();
}

template <typename T>
int split_ba(const SplitParams& p, xk_dtype bdt, hipStream_t s) {
  switch (bdt) {
    case XK_F32: return launch_split<T, float>(p, s);
    case XK_BF16: return launch_split<T, bf16>(p, s);
    case XK_F16: return launch_split<T, f16>(p, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}

}  // namespace
}  // namespace xk

using namespace xk;

extern "C" int xk_fused_qkvzba_split_reshape_cat(
    const void* mixed_qkvz, int64_t stride_qkvz_row, const void* mixed_ba,
    int64_t stride_ba_row, void* mixed_qkv, void* z, void* b, void* a, int64_t rows,
    int64_t num_heads_qk, int64_t num_heads_v, int64_t head_qk, int64_t head_v,
    xk_dtype dtype, xk_dtype ba_dtype, void* stream) {
  if (rows < 0 || num_heads_qk <= 0 || num_heads_v <= 0 || head_qk <= 0 || head_v <= 0 ||
      num_heads_v % num_heads_qk != 0)
    return XK_ERR_INVALID;
  const int64_t R = num_heads_v / num_heads_qk;
  const int64_t dt = 2 * head_qk + 2 * R * head_v;
  // Row widths are handled in int32 (a row of the projection).
  if (num_heads_qk * dt + 2 * num_heads_v > INT32_MAX / 2) return XK_ERR_UNSUPPORTED;
  if (stride_qkvz_row < num_heads_qk * dt || stride_ba_row < 2 * num_heads_v)
    return XK_ERR_INVALID;
  if (!is_float_dtype(dtype) || !is_float_dtype(ba_dtype)) return XK_ERR_UNSUPPORTED;
  if (rows == 0) return XK_OK;
  if (!mixed_qkvz || !mixed_ba || !mixed_qkv || !z || !b || !a) return XK_ERR_INVALID;
  SplitParams p{};
  p.qkvz = mixed_qkvz;
  p.sq = stride_qkvz_row;
  p.ba = mixed_ba;
  p.sba = stride_ba_row;
  p.qkv = mixed_qkv;
  p.z = z;
  p.b = b;
  p.a = a;
  p.rows = rows;
  p.nqk = static_cast<int>(num_heads_qk);
  p.nv = static_cast<int>(num_heads_v);
  p.hk = static_cast<int>(head_qk);
  p.hv = static_cast<int>(head_v);
  p.R = static_cast<int>(R);
  p.dt = static_cast<int>(dt);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case XK_F32: return split_ba<float>(p, ba_dtype, s);
    case XK_BF16: return split_ba<bf16>(p, ba_dtype, s);
    case XK_F16: return split_ba<f16>(p, ba_dtype, s);
    default: return XK_ERR_UNSUPPORTED;
  }
}
