// Internal launch interface of the page gather kernel (kv_gather.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvr {

// Copies the first seq_len tokens named by page_ids from a pool
// [num_pages][1][Hkv][page_size][head_dim] into out [Hkv][seq_len][head_dim].
// Moves 16-byte vectors when rows and pointers allow, else 4- or 2-byte ones.
hipError_t launch_gather_pages(const void* pool, const int32_t* page_ids, int num_kv_heads, int page_size, int head_dim,
                               int elem_size, int seq_len, void* out, hipStream_t stream);

// Copies every sequence's first seq_len tokens (seq_lens[b], or single_seq_len
// when seq_lens is null) from pools of page_size-token pages into pools of
// 16-token pages, pages16 per sequence at fixed stride (sequence b owns pages
// b * pages16 ..), and writes that layout's block table bt16
// [num_seqs][pages16].  head_dim * elem_size must be a multiple of 16 and
// every pointer 16-byte aligned.
hipError_t launch_repack_pages(const void* key_pool, const void* value_pool, const int32_t* block_tables,
                               int bt_stride, const int32_t* seq_lens, int single_seq_len, int num_seqs,
                               int num_kv_heads, int page_size, int head_dim, int elem_size, int pages16,
                               void* key16, void* value16, int32_t* bt16, hipStream_t stream);

} // namespace mvr
