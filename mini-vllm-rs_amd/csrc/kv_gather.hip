// Gather one request's KV pages into a contiguous [Hkv, L, D] tensor on the
// device: the GPU counterpart of reconstruct_contiguous_tensor
// (src/model_runner/server/kv_cache/paged_cache.rs:363-391), which narrows
// every page of the block table to its valid tokens and concatenates them on
// the token axis.  Pure data movement: the copy is bit-exact.
//
// HBM-bound: 2 * Hkv * L * D * elem_size bytes (read + write) per call.  Each
// thread moves one vector (16 bytes when a row allows it); consecutive threads
// walk one token row, so both the page reads and the contiguous writes are
// coalesced.  Any page size works: token t lives in page
// page_ids[t / page_size], slot t % page_size.
#include "kv_gather.hpp"

namespace mvr {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename V>
__global__ __launch_bounds__(256) void gather_pages_kernel(const V* __restrict__ pool, const int32_t* __restrict__ page_ids,
                                                           int num_kv_heads, int page_size, int row_vecs, int seq_len,
                                                           V* __restrict__ out, int64_t total_vecs) {
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < total_vecs; v += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(v % row_vecs); // vector within the row
    const int64_t ht = v / row_vecs;   // (head, token)
    const int t = (int)(ht % seq_len);
    const int h = (int)(ht / seq_len);
    const int64_t page = page_ids[t / page_size];
    const int slot = t % page_size;
    out[v] = pool[((page * num_kv_heads + h) * page_size + slot) * (int64_t)row_vecs + c];
  }
}

template <typename V>
hipError_t launch_typed(const void* pool, const int32_t* page_ids, int num_kv_heads, int page_size, int row_bytes,
                        int seq_len, void* out, hipStream_t stream) {
  const int row_vecs = row_bytes / (int)sizeof(V);
  const int64_t total = (int64_t)num_kv_heads * seq_len * row_vecs;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64; // grid-stride beyond 64 blocks per CU
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(gather_pages_kernel<V>, dim3((unsigned)blocks), dim3(256), 0, stream, static_cast<const V*>(pool),
                     page_ids, num_kv_heads, page_size, row_vecs, seq_len, static_cast<V*>(out), total);
  return hipGetLastError();
}

} // namespace

hipError_t launch_gather_pages(const void* pool, const int32_t* page_ids, int num_kv_heads, int page_size, int head_dim,
                               int elem_size, int seq_len, void* out, hipStream_t stream) {
  const int row_bytes = head_dim * elem_size;
  const uintptr_t align = (uintptr_t)pool | (uintptr_t)out;
  if (row_bytes % 16 == 0 && align % 16 == 0)
    return launch_typed<u32x4>(pool, page_ids, num_kv_heads, page_size, row_bytes, seq_len, out, stream);
  if (row_bytes % 4 == 0 && align % 4 == 0)
    return launch_typed<uint32_t>(pool, page_ids, num_kv_heads, page_size, row_bytes, seq_len, out, stream);
  return launch_typed<uint16_t>(pool, page_ids, num_kv_heads, page_size, row_bytes, seq_len, out, stream);
}

} // namespace mvr
