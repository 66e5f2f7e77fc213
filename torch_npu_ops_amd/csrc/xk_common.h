// Shared device helpers for the gfx950 kernels: element conversion, vector
// memory access and wave64 / work-group reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "xk_ops.h"

namespace xk {

using bf16 = __bf16;
using f16 = _Float16;

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Scalar conversion.  bf16/f16 -> f32 is exact; f32 -> bf16/f16 rounds to
// nearest even (gfx950 has a native v_cvt_pk_bf16_f32 for the bf16 case).
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ float to_f32(T v) {
  return static_cast<float>(v);
}
template <typename T>
__device__ __forceinline__ T from_f32(float v) {
  return static_cast<T>(v);
}

// Load one element whose dtype is only known at run time (used for small
// parameter vectors such as weights and gates, never in a bandwidth loop).
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i,
                                             xk_dtype dt) {
  switch (dt) {
    case XK_BF16:
      return static_cast<float>(reinterpret_cast<const bf16*>(p)[i]);
    case XK_F16:
      return static_cast<float>(reinterpret_cast<const f16*>(p)[i]);
    default:
      return reinterpret_cast<const float*>(p)[i];
  }
}

// ---------------------------------------------------------------------------
// Vector access: N consecutive elements moved as one aligned load/store.
// ---------------------------------------------------------------------------
template <typename T, int N>
struct alignas(sizeof(T) * N) Vec {
  T v[N];
};

// Streaming (read-once / write-once) vector access: non-temporal hints keep
// streamed tensors from displacing reusable lines in L2 and the Infinity
// Cache.  Vectors of 4, 8 or 16 bytes; other sizes fall back to plain
// accesses.
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <int BYTES> struct RawOf { using type = void; };
template <> struct RawOf<4> { using type = unsigned int; };
template <> struct RawOf<8> { using type = u32x2; };
template <> struct RawOf<16> { using type = u32x4; };

template <typename V>
__device__ __forceinline__ V ld_stream(const V* p) {
  using U = typename RawOf<sizeof(V)>::type;
  if constexpr (std::is_void<U>::value) {
    return *p;
  } else {
    return __builtin_bit_cast(V, __builtin_nontemporal_load(reinterpret_cast<const U*>(p)));
  }
}
template <typename V>
__device__ __forceinline__ void st_stream(V* p, const V& v) {
  using U = typename RawOf<sizeof(V)>::type;
  if constexpr (std::is_void<U>::value) {
    *p = v;
  } else {
    __builtin_nontemporal_store(__builtin_bit_cast(U, v), reinterpret_cast<U*>(p));
  }
}

// Register array with no alignment requirement (any N).
template <typename T, int N>
struct Arr {
  T v[N];
};

template <typename T, int N>
__device__ __forceinline__ void load_vec_f32(const T* p, float (&out)[N]) {
  Vec<T, N> t = *reinterpret_cast<const Vec<T, N>*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) out[i] = to_f32(t.v[i]);
}

template <typename T, int N>
__device__ __forceinline__ void store_vec_f32(T* p, const float (&in)[N]) {
  Vec<T, N> t;
#pragma unroll
  for (int i = 0; i < N; ++i) t.v[i] = from_f32<T>(in[i]);
  *reinterpret_cast<Vec<T, N>*>(p) = t;
}

// ---------------------------------------------------------------------------
// Reductions.
// ---------------------------------------------------------------------------
// One DPP move of a float (every row and bank enabled).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Lane l's value, broadcast (v_readlane).
__device__ __forceinline__ float readlane_f32(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

// Sum over aligned groups of `width` lanes (width a power of two <= 64),
// every lane of a group receiving the sum; every lane of a group must be
// active.  Within a 16-lane row the butterfly runs on DPP moves (quad
// permutations, then the half-row and row mirrors), a few cycles each where
// a ds_bpermute shuffle is an LDS round trip; rows combine through
// v_readlane.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(WIDTH >= 1 && WIDTH <= 64 && (WIDTH & (WIDTH - 1)) == 0, "power of two <= 64");
  if constexpr (WIDTH >= 2) v += dpp_f32<0xB1>(v);   // quad_perm(1,0,3,2): lane ^ 1
  if constexpr (WIDTH >= 4) v += dpp_f32<0x4E>(v);   // quad_perm(2,3,0,1): lane ^ 2
  if constexpr (WIDTH >= 8) v += dpp_f32<0x141>(v);  // row_half_mirror: quad pairs
  if constexpr (WIDTH >= 16) v += dpp_f32<0x140>(v); // row_mirror: half-row pairs
  if constexpr (WIDTH >= 32) {
    const float a = readlane_f32(v, 0) + readlane_f32(v, 16);
    const float b = readlane_f32(v, 32) + readlane_f32(v, 48);
    v = WIDTH == 64 ? a + b : ((threadIdx.x & 32) ? b : a);
  }
  return v;
}

// Hardware reciprocal (v_rcp_f32, ~1 ulp): sigmoid/SiLU feed bf16/fp16 or
// tolerance-checked fp32 outputs, so the IEEE division sequence (about ten
// instructions) is not needed.  exp(-x) overflowing to +inf gives rcp = 0,
// the correct limit.
__device__ __forceinline__ float fast_rcp(float x) {
  return __builtin_amdgcn_rcpf(x);
}

// Hardware reciprocal square root (v_rsq_f32, within ~1 ulp), for norm
// scales of positive arguments (a sum of squares plus eps): one instruction
// where 1.0f / sqrtf(x) is an IEEE square root and an IEEE division
// sequence.
__device__ __forceinline__ float rsqrt_hw(float x) { return __builtin_amdgcn_rsqf(x); }

__device__ __forceinline__ float sigmoid(float x) {
  return fast_rcp(1.0f + __expf(-x));
}

__device__ __forceinline__ float silu(float x) { return x * sigmoid(x); }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? XK_OK : static_cast<int>(e);
}

inline bool aligned(const void* p, int bytes) {
  return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) {
  return (a + b - 1) / b;
}

// Compute units of the current device (cached per device; 256 if the
// query fails).
inline int num_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev] = n;
  }
  return cached[dev];
}

inline int elem_bytes(xk_dtype dt) {
  switch (dt) {
    case XK_BF16:
    case XK_F16:
      return 2;
    case XK_I64:
      return 8;
    default:
      return 4;
  }
}

inline bool is_float_dtype(xk_dtype dt) {
  return dt == XK_F32 || dt == XK_BF16 || dt == XK_F16;
}

}  // namespace xk
