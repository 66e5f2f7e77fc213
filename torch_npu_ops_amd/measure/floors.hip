// Reference kernels for bench.py's floors: an empty kernel (the launch
// floor), a plain device copy (the floor of an HBM-bound kernel that
// moves the same bytes), an in-place read-modify-write of the last bytes
// of every row (the floor of a kernel with that strided pattern) and a
// copy by (64-row, one-head) tiles (the pattern of the chunked-GDN stage
// kernels).  Measurement only: built into libxk_measure.so,
// loaded by bench.py, and not part of the C-ABI in include/xk_ops.h.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ void empty_kernel() {}

// One 16-byte vector per lane, non-temporal in and out: the access pattern
// of the row kernels it is compared with.
__global__ void __launch_bounds__(256) copy16_kernel(const u32x4* __restrict__ src,
                                                     u32x4* __restrict__ dst, int64_t n16) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// The last `tail` bytes of each of `rows` rows of `pitch` bytes, read and
// written back changed, one 16-byte vector per lane (lpr lanes per row).
__global__ void __launch_bounds__(256) tail_rw_kernel(char* x, int64_t rows, int64_t pitch,
                                                      int64_t tail, int lpr) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= rows * lpr) return;
  u32x4* p = reinterpret_cast<u32x4*>(x + (i / lpr) * pitch + (pitch - tail) + 16 * (i % lpr));
  *p = *p ^ 1u;
}

// Tile copy with the access pattern of the chunked-GDN stage kernels: a
// [rows, slices * width] array read and written as tiles of 64 rows x one
// `width`-byte slice (a (chunk, head) piece of a [T, H, D] tensor), one
// block per tile, blocks taking the slices of one row group before the
// next; each lane moves `width * 64 / 4096` 16-byte vectors, all loads
// issued before the stores.
template <int V16>
__global__ void __launch_bounds__(256) tile_copy_kernel(const char* __restrict__ src,
                                                        char* __restrict__ dst, int64_t rows,
                                                        int slices, int width) {
  const int64_t b = blockIdx.x;
  const int slice = static_cast<int>(b % slices);
  const int64_t r0 = (b / slices) * 64;
  const int lpr = width / 16;  // lanes per row
  const int64_t pitch = static_cast<int64_t>(slices) * width;
  u32x4 v[V16];
#pragma unroll
  for (int j = 0; j < V16; ++j) {
    const int idx = j * 256 + threadIdx.x;
    const int64_t r = r0 + idx / lpr;
    v[j] = r < rows ? *reinterpret_cast<const u32x4*>(src + r * pitch + slice * width + 16 * (idx % lpr))
                    : u32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int j = 0; j < V16; ++j) {
    const int idx = j * 256 + threadIdx.x;
    const int64_t r = r0 + idx / lpr;
    if (r < rows) *reinterpret_cast<u32x4*>(dst + r * pitch + slice * width + 16 * (idx % lpr)) = v[j];
  }
}

}  // namespace

// Tile copy floor: rows x (slices * width) bytes read and written in tiles
// of 64 rows x width bytes (width 256 or 512: 4 or 8 vectors per lane).
extern "C" int xkm_tile_copy(const void* src, void* dst, int64_t rows, int slices, int width,
                             void* stream) {
  if (rows <= 0 || slices <= 0 || (width != 256 && width != 512)) return -1;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0) return -1;
  const int64_t blocks = (rows + 63) / 64 * slices;
  if (blocks > INT32_MAX) return -1;
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (width == 256)
    hipLaunchKernelGGL(tile_copy_kernel<4>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                       static_cast<const char*>(src), static_cast<char*>(dst), rows, slices, width);
  else
    hipLaunchKernelGGL(tile_copy_kernel<8>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s,
                       static_cast<const char*>(src), static_cast<char*>(dst), rows, slices, width);
  return static_cast<int>(hipGetLastError());
}

extern "C" int xkm_empty(void* stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream));
  return static_cast<int>(hipGetLastError());
}

// Copies `bytes` (a multiple of 16; both pointers 16-byte aligned): reads
// `bytes` and writes `bytes`.
extern "C" int xkm_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  if (bytes <= 0 || bytes % 16 != 0) return -1;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0) return -1;
  const int64_t n16 = bytes / 16;
  const int64_t blocks = (n16 + 255) / 256;
  if (blocks > INT32_MAX) return -1;
  hipLaunchKernelGGL(copy16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const u32x4*>(src),
                     static_cast<u32x4*>(dst), n16);
  return static_cast<int>(hipGetLastError());
}

// Strided in-place floor: rows x tail bytes at the end of rows of `pitch`
// bytes (tail and pitch multiples of 16, tail <= pitch, x 16-byte aligned);
// reads and writes rows * tail bytes.
extern "C" int xkm_tail_rw(void* x, int64_t rows, int64_t pitch, int64_t tail, void* stream) {
  if (rows <= 0 || tail <= 0 || tail > pitch || tail % 16 != 0 || pitch % 16 != 0) return -1;
  if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || tail / 16 > 1024) return -1;
  const int lpr = static_cast<int>(tail / 16);
  const int64_t blocks = (rows * lpr + 255) / 256;
  if (blocks > INT32_MAX) return -1;
  hipLaunchKernelGGL(tail_rw_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<char*>(x), rows, pitch, tail,
                     lpr);
  return static_cast<int>(hipGetLastError());
}
