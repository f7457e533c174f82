// Internal launch interface of the chunked-prefill kernel (paged_prefill.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mvr {

// Rows per block of the prefill kernel (4 wavefronts x 32 grouped rows).
constexpr int kPrefillBlockRows = 128;

struct PrefillParams {
  const void* q;
  int64_t q_stride_head, q_stride_token;
  const void* key_pool;
  const void* value_pool;
  const int32_t* block_tables;
  int32_t block_table_stride;
  const int32_t* seq_lens;  // may be null: single_seq_len
  const int32_t* cu_q_lens; // may be null: single_q_len
  int32_t single_seq_len, single_q_len;
  void* out;
  int64_t out_stride_head, out_stride_token;
  float* partial_o;  // [slots][128][head_dim] fp32 when kv_splits > 1
  float* partial_ml; // [slots][128][2]
  // page_size: a multiple of 16, or one that prefill_token_pages_supported
  // accepts (read in place by the token-page kernels).
  int32_t num_seqs, num_kv_heads, group_size, page_size;
  // Page of a token without a divide: page = tok * page_magic >> page_magic_shift
  // for every tok in [0, 2^31) (page_divider).
  uint64_t page_magic;
  int32_t page_magic_shift;
  int32_t row_tiles;  // 128-row tiles per (sequence, kv head)
  int32_t kv_splits; // key-range splits per row tile
  float scale_log2;
  // Cascade prefix pass (optional): keys [0, key_end[b]) only, all visible to
  // every row; results as normalised fp32 rows + log2-sum-exp.
  const int32_t* key_end;
  float* state_o;   // [q head][state_tokens][D]
  float* state_lse; // [q head][state_tokens]
  int32_t state_tokens;
  // Sequences b in [skip_seq_lo, skip_seq_hi] with q_len <= skip_q_max (0:
  // none) belong to another launch of the same call and are skipped.
  int32_t skip_seq_lo, skip_seq_hi, skip_q_max;
  // Main grid: one block per (sequence, kv head, row tile, key split) for the
  // sequences [seq_lo, seq_lo + seq_count) (count 0: every sequence).  Partial
  // slot of (b, h, rt, split): (((b - seq_lo) * num_kv_heads + h) * row_tiles
  // + rt) * kv_splits + split.
  int32_t seq_lo, seq_count;
  // Catch-up blocks after the main grid: one per sequence of [catch_lo,
  // catch_lo + catch_count) outside the main range, each computing every
  // (kv head, row tile) of its sequence unsplit (normally none has rows: they
  // cover sequences that host hints placed in another launch's class).
  int32_t catch_lo, catch_count;
  int32_t groups; // wavefront groups of 4 per block: 2, or 1 (always 1 for head_dim > 128)
};

// Division by the invariant page_size as a multiply and a shift, the
// round-up method of Granlund and Montgomery ("Division by invariant integers
// using multiplication", PLDI 1994, theorem 4.2): with l = ceil(log2 d),
// shift = 32 + l and magic = ceil(2^shift / d), 2^shift <= magic * d <=
// 2^shift + 2^l, so floor(n * magic / 2^shift) = floor(n / d) for every n <
// 2^32; magic < 2^33 + 1 keeps n * magic below 2^64 for n < 2^31.
inline void page_divider(int32_t d, uint64_t& magic, int32_t& shift) {
  int l = 0;
  while ((1ll << l) < d) l++;
  shift = 32 + l;
  magic = (uint64_t)((((unsigned __int128)1 << shift) + (unsigned)d - 1) / (unsigned)d);
}

// Head dimensions the prefill kernel takes: every multiple of 32 up to 256
// (F16 in 64-token key tiles, F32 in 32-token tiles; rows of more than 128
// elements in blocks of one wavefront group, one wavefront per SIMD).
constexpr bool prefill_head_dim_supported(int d) { return d >= 32 && d <= 256 && d % 32 == 0; }

// Tokens that one 64-lane direct-to-LDS load of the prefill kernel covers
// (16 bytes per lane, whole token rows at head_dim 64 and 128).
constexpr int prefill_tokens_per_load(int d, int elem_bytes) { return 64 * 16 / (d * elem_bytes); }

// Page sizes that are not a multiple of 16 which the prefill kernel reads in
// place (token pages): head_dim 64 and 128, page sizes that are a multiple
// of the tokens per load (so that every load's tokens lie in one page:
// F16 D=128 multiples of 4, F16 D=64 of 8, F32 D=128 of 2, F32 D=64 of 4),
// and pages (all KV heads) of less than 4 GiB, whose byte offsets the
// kernel keeps in 32 bits.
constexpr bool prefill_token_pages_supported(int page_size, int num_kv_heads, int d, int elem_bytes) {
  return (d == 64 || d == 128) && page_size >= 2 && page_size % prefill_tokens_per_load(d, elem_bytes) == 0 &&
         (long long)num_kv_heads * page_size * d * elem_bytes < (1LL << 32);
}

// f32: F32 Q/K/V/out (v_mfma_f32_32x32x2_f32); otherwise F16.
hipError_t launch_paged_prefill(const PrefillParams& params, int head_dim, bool f32, hipStream_t stream);

} // namespace mvr
