// Fused rotary embedding + KV-page append for gfx950 (MI355X, CDNA4).
//
// Replaces, for every request of a layer in one launch, the steps
// forward_attention runs before each attention call
// (src/models/backends/common.rs:294-320): forward_rope on the request's Q
// and K (common.rs:344-359, candle-nn's rope / rope_i) and
// append_new_key_value (src/model_runner/server/kv_cache/paged_cache.rs:
// 170-199, :290-327; physical_page_pool.rs:188-209), which copies the new
// K/V rows into their page slots.  Here the page allocation stays on the
// host (the block table already holds the pages), and the kernel writes the
// rotated K and the V rows straight through the block table.
//
// One block row (blockIdx.x) per packed token: the block finds its request
// from cu_q_lens and its page by one block-table entry.  Each thread handles
// one 8-element item of one row:
// the query heads (rotated to q_out), the KV heads (rotated into the key
// pool) and the KV heads again (copied into the value pool).  Items of a row
// are adjacent lanes, so every row is read and written with coalesced 8- or
// 16-byte accesses.  HBM-bound: per token (Hq + Hkv)*D*es*2 + Hkv*D*es*2
// bytes plus one cos/sin row.
//
// Arithmetic follows the reference in the activation dtype: each product and
// the sum is rounded to T, with no fused multiply-add (contraction is off for
// this file).  F16 rounds each f32 result to f16: an f16 x f16 product is
// exact in f32, and rounding an f32 sum of two f16 values to f16 gives the
// correctly rounded f16 sum, as the half crate's per-operation rounding does.
#include "kv_append.hpp"

// No contraction anywhere in this file: the compiler narrows the F16
// arithmetic to f16 instructions (exact here) but would then fuse a product
// into the following add as v_pk_fma_f16 (v_fma_f32 for F32), dropping the
// product's rounding.  Library helpers such as __fmul_rn are inlined with
// contraction allowed, so the arithmetic below uses plain operators.
#pragma clang fp contract(off)

namespace mvr {
namespace {

typedef _Float16 half_t;
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(4))) int32_t const_i32;

constexpr int kThreads = 256;
constexpr int kItem = 8; // elements (4 rotation pairs) per thread item

template <typename T>
struct Arith;

template <>
struct Arith<float> {
  typedef float4v vec;
  __device__ static float mul(float a, float b) { return a * b; }
  __device__ static float add(float a, float b) { return a + b; }
  __device__ static float sub(float a, float b) { return a - b; }
  __device__ static float4v load(const float* p) { return *reinterpret_cast<const float4v*>(p); }
  __device__ static void store(float* p, float4v v) { *reinterpret_cast<float4v*>(p) = v; }
  __device__ static float get(float4v v, int e) { return v[e]; }
};

template <>
struct Arith<half_t> {
  typedef half4 vec;
  __device__ static float r(float x) { return (float)(half_t)x; }
  __device__ static float mul(float a, float b) { return r(a * b); }
  __device__ static float add(float a, float b) { return r(a + b); }
  __device__ static float sub(float a, float b) { return r(a - b); }
  __device__ static half4 load(const half_t* p) { return *reinterpret_cast<const half4*>(p); }
  __device__ static void store(half_t* p, half4 v) { *reinterpret_cast<half4*>(p) = v; }
  __device__ static float get(half4 v, int e) { return (float)v[e]; }
};

// Rotates the 4 pairs of one item (common.rs:355-358): lo and hi hold the
// item's elements at lo_off and hi_off of its row (Neox pairs (i, i + D/2),
// Interleaved pairs (2i, 2i + 1), i = 4j .. 4j + 3); the results go back to
// ylo and yhi in the same places.
template <typename T, int ROPE>
__device__ __forceinline__ void rotate_item(const typename Arith<T>::vec& lo, const typename Arith<T>::vec& hi,
                                            const typename Arith<T>::vec& c, const typename Arith<T>::vec& s,
                                            typename Arith<T>::vec& ylo, typename Arith<T>::vec& yhi) {
  typedef Arith<T> A;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    float a, b;
    if (ROPE == 0) {
      a = A::get(lo, e);
      b = A::get(hi, e);
    } else {
      a = e < 2 ? A::get(lo, 2 * e) : A::get(hi, 2 * e - 4);
      b = e < 2 ? A::get(lo, 2 * e + 1) : A::get(hi, 2 * e - 3);
    }
    const float ce = A::get(c, e), se = A::get(s, e);
    const float ya = A::sub(A::mul(a, ce), A::mul(b, se));
    const float yb = A::add(A::mul(a, se), A::mul(b, ce));
    if (ROPE == 0) {
      ylo[e] = (T)ya;
      yhi[e] = (T)yb;
    } else if (e < 2) {
      ylo[2 * e] = (T)ya;
      ylo[2 * e + 1] = (T)yb;
    } else {
      yhi[2 * e - 4] = (T)ya;
      yhi[2 * e - 3] = (T)yb;
    }
  }
}

// One item per thread: blockIdx.y * kThreads + threadIdx.x over the token's
// (Hq + 2 Hkv) * D/8 items.  The item's source elements depend on the token
// only, so they are loaded first and their latency overlaps the lookup of the
// token's request, position and page, a chain of dependent loads: cu_q_lens
// (one vector load and a ballot for up to 63 requests, a binary search
// beyond), seq_lens, then the rotary rows and the block-table entry.
template <typename T, int ROPE>
__global__ __launch_bounds__(kThreads) void rope_append_kernel(RopeAppendParams p) {
  typedef Arith<T> A;
  typedef typename A::vec V;
  const int n = blockIdx.x; // packed token
  const int D = p.head_dim;
  const int items_per_row = D / kItem;
  const int items = (p.num_q_heads + 2 * p.num_kv_heads) * items_per_row;
  const int it = blockIdx.y * kThreads + threadIdx.x;
  const bool active = it < items;
  const int row = active ? it / items_per_row : 0;
  const int j = it - row * items_per_row;
  const int kind = row < p.num_q_heads ? 0 : row < p.num_q_heads + p.num_kv_heads ? 1 : 2; // Q, K, V
  const int h = kind == 0 ? row : kind == 1 ? row - p.num_q_heads : row - p.num_q_heads - p.num_kv_heads;
  const int lo_off = kind == 2 ? kItem * j : ROPE == 0 ? 4 * j : 8 * j;
  const int hi_off = kind == 2 ? kItem * j + 4 : ROPE == 0 ? D / 2 + 4 * j : 8 * j + 4;
  const T* src = kind == 0 ? static_cast<const T*>(p.q) + h * p.q_stride_head + (int64_t)n * p.q_stride_token
               : kind == 1 ? static_cast<const T*>(p.k) + h * p.k_stride_head + (int64_t)n * p.k_stride_token
                           : static_cast<const T*>(p.v) + h * p.v_stride_head + (int64_t)n * p.v_stride_token;
  V lo{}, hi{};
  if (active) {
    lo = A::load(src + lo_off);
    hi = A::load(src + hi_off);
  }

  int b = 0, q_start = 0, q_len = p.total_q;
  if (p.cu_q_lens) {
    // Largest b with cu_q_lens[b] <= n (uniform per block).
    if (p.num_seqs < 64) {
      const int l = threadIdx.x & 63;
      const int cu_l = l <= p.num_seqs ? p.cu_q_lens[l] : INT32_MAX;
      const uint64_t le = __ballot(cu_l <= n);
      b = max(__builtin_amdgcn_readfirstlane(__popcll(le)) - 1, 0); // cu_q_lens[0] = 0 <= n: at least one
      q_start = __builtin_amdgcn_readlane(cu_l, b);
      q_len = __builtin_amdgcn_readlane(cu_l, b + 1) - q_start;
    } else {
      const const_i32* cu = (const const_i32*)p.cu_q_lens;
      int lo_b = 0, hi_b = p.num_seqs - 1;
      while (lo_b < hi_b) {
        const int mid = (lo_b + hi_b + 1) >> 1;
        if (cu[mid] <= n)
          lo_b = mid;
        else
          hi_b = mid - 1;
      }
      b = lo_b;
      q_start = cu[b];
      q_len = cu[b + 1] - q_start;
    }
  }
  const int seq_len = p.seq_lens ? ((const const_i32*)p.seq_lens)[b] : p.single_seq_len;
  const int pos = seq_len - q_len + (n - q_start); // cached_kv_len + i (kv_cache/utils.rs:20-24)
  // Positions outside [0, max_seq_len) only come from tables that break the
  // contract (seq_len < q_len or > max_seq_len): write nothing rather than
  // leave the block-table row, the rotary tables or the pools.
  if (pos < 0 || pos >= p.single_seq_len || !active) return;
  const const_i32* bt = (const const_i32*)p.block_tables + (int64_t)b * p.block_table_stride;
  const int64_t page = bt[pos / p.page_size];
  const int slot = pos % p.page_size;
  T* dst = kind == 0 ? static_cast<T*>(p.q_out) + h * p.q_out_stride_head + (int64_t)n * p.q_out_stride_token
         : kind == 1 ? static_cast<T*>(p.key_pool) + ((page * p.num_kv_heads + h) * p.page_size + slot) * D
                     : static_cast<T*>(p.value_pool) + ((page * p.num_kv_heads + h) * p.page_size + slot) * D;
  if (kind == 2) {
    A::store(dst + lo_off, lo);
    A::store(dst + hi_off, hi);
    return;
  }
  const T* cos_row = static_cast<const T*>(p.cos_table) + (int64_t)pos * (D / 2);
  const T* sin_row = static_cast<const T*>(p.sin_table) + (int64_t)pos * (D / 2);
  const V c = A::load(cos_row + 4 * j);
  const V sn = A::load(sin_row + 4 * j);
  V ylo, yhi;
  rotate_item<T, ROPE>(lo, hi, c, sn, ylo, yhi);
  A::store(dst + lo_off, ylo);
  A::store(dst + hi_off, yhi);
}

template <typename T, int ROPE>
hipError_t launch_typed(const RopeAppendParams& p, hipStream_t stream) {
  const int items = (p.num_q_heads + 2 * p.num_kv_heads) * (p.head_dim / kItem);
  const int gy = (items + kThreads - 1) / kThreads;
  hipLaunchKernelGGL((rope_append_kernel<T, ROPE>), dim3((unsigned)p.total_q, (unsigned)gy), dim3(kThreads), 0,
                     stream, p);
  return hipGetLastError();
}

} // namespace

hipError_t launch_rope_append(const RopeAppendParams& params, int dtype, int rope_type, hipStream_t stream) {
  if (dtype == 1) return rope_type == 0 ? launch_typed<half_t, 0>(params, stream) : launch_typed<half_t, 1>(params, stream);
  return rope_type == 0 ? launch_typed<float, 0>(params, stream) : launch_typed<float, 1>(params, stream);
}

} // namespace mvr
