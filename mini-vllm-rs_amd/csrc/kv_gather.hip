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
// page_ids[t / page_size], slot t % page_size.  The same file repacks a
// batch's pages into 16-token pages for attention calls whose page size is
// not a multiple of 16.
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

// Repack of a batch's pages into 16-token pages (pages16 per sequence, fixed
// stride): sequence b's token t moves to page b * pages16 + t / 16, slot
// t % 16, of a new pool [num_seqs * pages16][1][Hkv][16][D], and the new block
// table row b is b * pages16 + 0, 1, ...  Tokens past seq_lens[b] are not
// copied (attention never reads them as keys).  Element v walks vectors of a
// row fastest, then tokens, so reads and writes of consecutive slots are
// contiguous.
template <typename V>
__global__ __launch_bounds__(256) void repack_pages_kernel(const V* __restrict__ kpool, const V* __restrict__ vpool,
                                                           const int32_t* __restrict__ block_tables, int bt_stride,
                                                           const int32_t* __restrict__ seq_lens, int single_seq_len,
                                                           int num_kv_heads, int page_size, int row_vecs, int pages16,
                                                           V* __restrict__ k16, V* __restrict__ v16,
                                                           int32_t* __restrict__ bt16, int64_t total_vecs) {
  const int tokens16 = pages16 * 16;
  for (int64_t v = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; v < total_vecs; v += (int64_t)gridDim.x * blockDim.x) {
    const int c = (int)(v % row_vecs);
    int64_t rest = v / row_vecs;
    const int t = (int)(rest % tokens16);
    rest /= tokens16;
    const int h = (int)(rest % num_kv_heads);
    const int b = (int)(rest / num_kv_heads);
    if (c == 0 && h == 0 && t % 16 == 0) bt16[(int64_t)b * pages16 + t / 16] = b * pages16 + t / 16;
    const int L = seq_lens ? seq_lens[b] : single_seq_len;
    if (t >= L || t / page_size >= bt_stride) continue; // the second only if a seq_len breaks the table's bound
    const int64_t page = block_tables[(int64_t)b * bt_stride + t / page_size];
    const int64_t src = ((page * num_kv_heads + h) * page_size + t % page_size) * (int64_t)row_vecs + c;
    const int64_t dst = ((((int64_t)b * pages16 + t / 16) * num_kv_heads + h) * 16 + t % 16) * (int64_t)row_vecs + c;
    k16[dst] = kpool[src];
    v16[dst] = vpool[src];
  }
}

} // namespace

hipError_t launch_repack_pages(const void* key_pool, const void* value_pool, const int32_t* block_tables,
                               int bt_stride, const int32_t* seq_lens, int single_seq_len, int num_seqs,
                               int num_kv_heads, int page_size, int head_dim, int elem_size, int pages16,
                               void* key16, void* value16, int32_t* bt16, hipStream_t stream) {
  typedef u32x4 V; // rows of a multiple of 32 F16/F32 elements: whole 16-byte vectors, pointers checked 16-byte aligned
  const int row_vecs = head_dim * elem_size / (int)sizeof(V);
  const int64_t total = (int64_t)num_seqs * num_kv_heads * pages16 * 16 * row_vecs;
  int64_t blocks = (total + 255) / 256;
  if (blocks > 256 * 64) blocks = 256 * 64;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(repack_pages_kernel<V>, dim3((unsigned)blocks), dim3(256), 0, stream,
                     static_cast<const V*>(key_pool), static_cast<const V*>(value_pool), block_tables, bt_stride,
                     seq_lens, single_seq_len, num_kv_heads, page_size, row_vecs, pages16, static_cast<V*>(key16),
                     static_cast<V*>(value16), bt16, total);
  return hipGetLastError();
}

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
