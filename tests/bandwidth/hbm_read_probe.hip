// HBM read ceilings of the part, measured with the access patterns the
// attention kernels are judged against (test and measurement infrastructure,
// not part of the library):
//   * hbm_stream_read: one linear pass over a buffer, 16-byte loads, four in
//     flight per thread over a grid-stride loop;
//   * hbm_page_walk_read: the same bytes as 4 KiB pages (16 tokens x 128 dims
//     x 2 bytes, one KV head's slab of one page) visited in a given order,
//     one wavefront per page and four pages in flight per wavefront, as a
//     paged K/V walk reads them.
// Each thread sums what it reads and writes one float, so nothing is elided.
// Bounds: the host checks that bytes is a multiple of 4 KiB, that every page
// id lies in [0, bytes / 4 KiB) and that out holds grid * 256 floats.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kPageVecs = 4096 / 16; // 16-byte vectors per 4 KiB page

__global__ __launch_bounds__(kThreads) void stream_read_kernel(const f4* __restrict__ in, size_t n16, float* out) {
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  const size_t stride = (size_t)gridDim.x * kThreads;
  size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  for (; i + 3 * stride < n16; i += 4 * stride) acc += in[i] + in[i + stride] + in[i + 2 * stride] + in[i + 3 * stride];
  for (; i < n16; i += stride) acc += in[i];
  out[(size_t)blockIdx.x * kThreads + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

__global__ __launch_bounds__(kThreads) void page_walk_kernel(const f4* __restrict__ in, const int32_t* __restrict__ order,
                                                             int n_pages, float* out) {
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * kThreads + threadIdx.x) >> 6);
  const int n_waves = (int)(gridDim.x * (kThreads / 64));
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  int p = wave;
  for (; p + 3 * n_waves < n_pages; p += 4 * n_waves) {
    f4 v[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const f4* pg = in + (size_t)order[p + k * n_waves] * kPageVecs;
#pragma unroll
      for (int j = 0; j < 4; j++) v[4 * k + j] = pg[lane + 64 * j];
    }
#pragma unroll
    for (int j = 0; j < 16; j++) acc += v[j];
  }
  for (; p < n_pages; p += n_waves) {
    const f4* pg = in + (size_t)order[p] * kPageVecs;
#pragma unroll
    for (int j = 0; j < 4; j++) acc += pg[lane + 64 * j];
  }
  out[(size_t)blockIdx.x * kThreads + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

} // namespace

extern "C" {

// Reads `bytes` (a multiple of 4 KiB) at `buf` once; out: grid * 256 floats.
int hbm_stream_read(const void* buf, size_t bytes, float* out, int grid, void* stream) {
  if (!buf || !out || bytes % 4096 || grid < 1) return -1;
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const f4*>(buf), bytes / 16, out);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Reads the n_pages 4 KiB pages of `buf` in the order given (device ids in
// [0, n_pages), checked by the caller); out: grid * 256 floats.
int hbm_page_walk_read(const void* buf, const int32_t* order, int n_pages, float* out, int grid, void* stream) {
  if (!buf || !order || !out || n_pages < 1 || grid < 1) return -1;
  hipLaunchKernelGGL(page_walk_kernel, dim3(grid), dim3(kThreads), 0, static_cast<hipStream_t>(stream),
                     static_cast<const f4*>(buf), order, n_pages, out);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

} // extern "C"
