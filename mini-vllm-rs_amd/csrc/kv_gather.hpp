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

} // namespace mvr
