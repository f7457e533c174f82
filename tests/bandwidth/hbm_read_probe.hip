// HBM read ceilings of the part, measured with the access patterns the
// attention kernels are judged against (test and measurement infrastructure,
// not part of the library):
//   * hbm_stream_read: one linear pass over a buffer, 16-byte loads, K in
//     flight per thread (K = 4, 8 or 16) over a grid-stride loop;
//   * hbm_page_walk_read: the same bytes as 4 KiB pages (16 tokens x 128 dims
//     x 2 bytes, one KV head's slab of one page) visited in a given order,
//     one wavefront per page and P pages in flight per wavefront (P = 2, 4
//     or 8), as a paged K/V walk reads them.
// Each thread sums what it reads and writes one float, so nothing is elided.
// Bounds: the host checks that bytes is a multiple of 4 KiB, that every page
// id lies in [0, bytes / 4 KiB) and that out holds grid * 256 floats.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256;
constexpr int kPageVecs = 4096 / 16; // 16-byte vectors per 4 KiB page

template <int K>
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const f4* __restrict__ in, size_t n16, float* out) {
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  const size_t stride = (size_t)gridDim.x * kThreads;
  size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
  for (; i + (K - 1) * stride < n16; i += K * stride) {
    f4 v[K];
#pragma unroll
    for (int k = 0; k < K; k++) v[k] = in[i + k * stride];
#pragma unroll
    for (int k = 0; k < K; k++) acc += v[k];
  }
  for (; i < n16; i += stride) acc += in[i];
  out[(size_t)blockIdx.x * kThreads + threadIdx.x] = acc[0] + acc[1] + acc[2] + acc[3];
}

template <int P>
__global__ __launch_bounds__(kThreads) void page_walk_kernel(const f4* __restrict__ in, const int32_t* __restrict__ order,
                                                             int n_pages, float* out) {
  const int lane = threadIdx.x & 63;
  const int wave = (int)((blockIdx.x * kThreads + threadIdx.x) >> 6);
  const int n_waves = (int)(gridDim.x * (kThreads / 64));
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  int p = wave;
  for (; p + (P - 1) * n_waves < n_pages; p += P * n_waves) {
    f4 v[4 * P];
#pragma unroll
    for (int k = 0; k < P; k++) {
      const f4* pg = in + (size_t)order[p + k * n_waves] * kPageVecs;
#pragma unroll
      for (int j = 0; j < 4; j++) v[4 * k + j] = pg[lane + 64 * j];
    }
#pragma unroll
    for (int j = 0; j < 4 * P; j++) acc += v[j];
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

// Reads `bytes` (a multiple of 4 KiB) at `buf` once with `inflight` (4, 8 or
// 16) loads in flight per thread; out: grid * 256 floats.
int hbm_stream_read(const void* buf, size_t bytes, float* out, int grid, int inflight, void* stream) {
  if (!buf || !out || bytes % 4096 || grid < 1) return -1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const f4* in = static_cast<const f4*>(buf);
  if (inflight == 4)
    hipLaunchKernelGGL(stream_read_kernel<4>, dim3(grid), dim3(kThreads), 0, st, in, bytes / 16, out);
  else if (inflight == 8)
    hipLaunchKernelGGL(stream_read_kernel<8>, dim3(grid), dim3(kThreads), 0, st, in, bytes / 16, out);
  else if (inflight == 16)
    hipLaunchKernelGGL(stream_read_kernel<16>, dim3(grid), dim3(kThreads), 0, st, in, bytes / 16, out);
  else
    return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Reads the n_pages 4 KiB pages of `buf` in the order given (device ids in
// [0, n_pages), checked by the caller), `inflight` (2, 4 or 8) pages in
// flight per wavefront; out: grid * 256 floats.
int hbm_page_walk_read(const void* buf, const int32_t* order, int n_pages, float* out, int grid, int inflight,
                       void* stream) {
  if (!buf || !order || !out || n_pages < 1 || grid < 1) return -1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const f4* in = static_cast<const f4*>(buf);
  if (inflight == 2)
    hipLaunchKernelGGL(page_walk_kernel<2>, dim3(grid), dim3(kThreads), 0, st, in, order, n_pages, out);
  else if (inflight == 4)
    hipLaunchKernelGGL(page_walk_kernel<4>, dim3(grid), dim3(kThreads), 0, st, in, order, n_pages, out);
  else if (inflight == 8)
    hipLaunchKernelGGL(page_walk_kernel<8>, dim3(grid), dim3(kThreads), 0, st, in, order, n_pages, out);
  else
    return -1;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

} // extern "C"
