// Page-wise attention kernels for gfx950 (MI355X, CDNA4).
//
// Replaces forward_paged_attention (src/models/backends/common.rs:739-817)
// and the GPU gather fallback (paged_cache.rs:363-391 + common.rs:703-737).
//
// Work decomposition: one wavefront per unit = (sequence b, kv head h, row
// tile rt, context partition).  A row tile holds 16*ROW_BLOCKS grouped query
// rows rho = r*q_len + i of kv head h (query head h*group_size + r, query
// position i), so every K/V element a wavefront reads from HBM feeds all the
// query heads that share it (GQA).  The context is walked in 16-token chunks
// read directly from the pools through the block table:
//   * K chunk -> registers in the MFMA A-operand layout (lane l holds token
//     l%16, 8 dims per 16-byte load), S^T = K Q^T with
//     v_mfma_f32_16x16x32_f16 (f16) or v_mfma_f32_16x16x4_f32 (f32);
//   * S^T lands with lane l owning query row l%16 and tokens 4*(l/16)+i, so
//     the online softmax (exp2 domain, fp32 state) needs only two cross-lane
//     max steps per chunk;
//   * V chunk -> 16-byte loads -> a swizzled LDS tile -> ds_read_b64_tr_b16
//     returns V^T in the A-operand layout, O^T += V^T P^T with
//     v_mfma_f32_16x16x16_f16 (f32: ds_read_b32 + v_mfma_f32_16x16x4_f32).
// Loads for chunk k+2 are issued before chunk k is consumed (two chunks in
// flight per wavefront; three for the plans that ask for a deep pipeline).  Partitions of one (b, h, rt) are merged by
// merge_partitions_kernel with the usual max / sum-of-exponentials rescale.
#include "paged_attention_kernels.hpp"

#include <math.h>

#include <atomic>

namespace mvr {
namespace {

typedef _Float16 half_t;
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) short4v lds_short4;
typedef __attribute__((address_space(4))) int32_t const_i32;

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ float wave_max_across_groups(float v) {
  // Lanes l, l^16, l^32, l^48 hold the same query row.
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ float wave_sum_across_groups(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}

// Per-sequence metadata (seq_lens / cu_q_lens may be absent for one request).
// Keys [key_begin, key_end) are this call's share of the context: all of it
// normally; the suffix after a shared prefix, or the prefix itself (where
// every row sees every prefix key), in the two passes of cascade attention.
struct SeqInfo {
  int seq_len, q_start, q_len, key_begin, key_end;
};

__device__ __forceinline__ SeqInfo load_seq(const PagedAttentionParams& p, int b) {
  SeqInfo s;
  // single_seq_len is the call's max_seq_len, whose pages the host has checked
  // to fit a block-table row: a larger device seq_len (a broken contract) is
  // clamped so that no read leaves the row or the planned partitions.
  s.seq_len = p.seq_lens ? min(p.seq_lens[b], p.single_seq_len) : p.single_seq_len;
  if (p.cu_q_lens) {
    s.q_start = p.cu_q_lens[b];
    s.q_len = p.cu_q_lens[b + 1] - s.q_start;
  } else {
    s.q_start = 0;
    s.q_len = p.single_q_len;
  }
  // Another launch's sequence: no rows here (every unit of it exits at once).
  if (s.q_len < p.class_q_min || (p.class_q_max > 0 && s.q_len > p.class_q_max)) s.q_len = 0;
  s.key_begin = p.key_begin ? p.key_begin[b] : 0;
  if (p.key_end) {
    s.key_end = p.key_end[b];
    s.seq_len = s.key_end + s.q_len; // every row's causal limit reaches past the prefix
  } else {
    s.key_end = s.seq_len;
  }
  return s;
}

// Causal limit of query i: key j visible iff j <= seq_len - q_len + i
// (common.rs:948-965), within this call's keys.
__device__ __forceinline__ int row_limit(const SeqInfo& s, int i) { return min(s.seq_len - s.q_len + i, s.key_end - 1); }

// Number of 16-token chunks row tile rt of a sequence must visit: keys up to
// the largest causal limit among its rows.
__device__ __forceinline__ int tile_chunks(const SeqInfo& s, int group_size, int rt, int tile_rows) {
  const int rows = group_size * s.q_len;
  const int rho0 = rt * tile_rows;
  if (rho0 >= rows || s.q_len <= 0) return 0;
  const int rho1 = min(rho0 + tile_rows, rows) - 1;
  const int max_i = (rho1 / s.q_len != rho0 / s.q_len) ? s.q_len - 1 : rho1 % s.q_len;
  const int last_key = row_limit(s, max_i); // -1: no key (a prefix pass over an empty prefix)
  return last_key < 0 ? 0 : last_key / kChunkTokens + 1;
}

// Partitions of a row tile: chunks [key_begin/16, n_chunks) in chunks_per_part pieces.
__device__ __forceinline__ int tile_parts(const SeqInfo& s, int n_chunks, int chunks_per_part) {
  const int kb = s.key_begin / kChunkTokens;
  return n_chunks > kb ? (n_chunks - kb + chunks_per_part - 1) / chunks_per_part : 0;
}

// Inclusive prefix sum over the 64 lanes of a wavefront.
__device__ __forceinline__ int wave_inclusive_sum(int v) {
  const int l = lane_id();
#pragma unroll
  for (int off = 1; off < kWaveSize; off <<= 1) {
    const int t = __shfl_up(v, off);
    if (l >= off) v += t;
  }
  return v;
}

// Dense layout of a ragged batch (one row tile per sequence and KV head):
// the live (sequence, partition) pairs are numbered from 0, 64 sequences at
// a time: first those sequences' full partitions (chunks_per_part chunks
// each), sequence by sequence, then each one's last, possibly partial,
// partition.  Work index w maps to (b, part); false once w is past every live
// pair.  Each wavefront derives its pair from the sequence lengths with one
// wave-wide scan per 64 sequences, so the grid needs no per-call table: it
// is sized for the worst case (max_parts per sequence) and its tail exits at
// once.  In-order dispatch then hands out the live units like a work queue,
// longest first within each 64 sequences, spread over all XCDs.
__device__ __forceinline__ SeqInfo lane_seq(const SeqInfo& s, int src) {
  return SeqInfo{__shfl(s.seq_len, src), __shfl(s.q_start, src), __shfl(s.q_len, src), __shfl(s.key_begin, src),
                 __shfl(s.key_end, src)};
}

// Also returns the sequence's SeqInfo (loaded by one lane of the scan), so the
// unit starts without a second round trip for it.
__device__ bool dense_unit(const PagedAttentionParams& p, int64_t w, int tile_rows, int& b_out, int& part_out,
                           SeqInfo& s_out) {
  const int l = lane_id();
  int64_t base = 0;
  for (int b0 = 0; b0 < p.num_seqs; b0 += kWaveSize) {
    const int b = b0 + l;
    int n = 0;
    SeqInfo s{0, 0, 0, 0, 0};
    if (b < p.num_seqs) {
      s = load_seq(p, b);
      n = tile_parts(s, tile_chunks(s, p.group_size, 0, tile_rows), p.chunks_per_part);
    }
    const int full = n > 0 ? n - 1 : 0, last = n > 0 ? 1 : 0;
    const int full_incl = wave_inclusive_sum(full), last_incl = wave_inclusive_sum(last);
    const int full_total = __shfl(full_incl, kWaveSize - 1), last_total = __shfl(last_incl, kWaveSize - 1);
    if (w < base + full_total) {
      const int64_t r = w - base;
      const uint64_t hit = __ballot(r >= full_incl - full && r < full_incl);
      const int src = __builtin_ctzll(hit);
      b_out = b0 + src;
      part_out = (int)(r - __shfl(full_incl - full, src));
      s_out = lane_seq(s, src);
      return true;
    }
    if (w < base + full_total + last_total) {
      const int64_t r = w - base - full_total;
      const uint64_t hit = __ballot(last == 1 && r == last_incl - 1);
      const int src = __builtin_ctzll(hit);
      b_out = b0 + src;
      part_out = __shfl(n, src) - 1;
      s_out = lane_seq(s, src);
      return true;
    }
    base += full_total + last_total;
  }
  return false;
}

// Cascade suffix pass: weights that merge this pass's normalised row (log2
// sum lb) with the prefix pass's state of the same row (srow):
//   out = (wa * o_a + wb * o_b) * inv.
// `has` is false when the row's sequence has no prefix (its prefix state was
// never written and must not be read).
struct PrefixWeights {
  bool has;
  float wa, wb, inv;
};
__device__ __forceinline__ PrefixWeights prefix_weights(const PagedAttentionParams& p, int b, int64_t srow, float lb) {
  if (!p.prefix_o || ((const const_i32*)p.seq_prefix_len)[b] <= 0) return {false, 0.f, 1.f, 1.f};
  const float la = p.prefix_lse[srow];
  const float mx = fmaxf(la, lb);
  const float wa = exp2f(la - mx), wb = exp2f(lb - mx);
  return {true, wa, wb, 1.f / (wa + wb)};
}

// ---------------------------------------------------------------------------
// dtype traits: how a 16-token chunk is loaded, multiplied and staged.
// ---------------------------------------------------------------------------

template <int D>
struct F16Traits {
  typedef half_t elem;
  static constexpr int kLoads = D / 32;   // 16-byte K loads (and V loads) per lane per chunk
  static constexpr int kQRegs = D / 32;   // half8 Q operand registers per row block
  typedef half8 kreg_t;
  typedef half8 vreg_t;
  typedef half8 qreg_t;

  // 16-row tiles: 3 wavefronts per SIMD; 32-row tiles: 2 (wider heads: 2, then 1).
  template <int NB>
  static constexpr int min_blocks() { return D <= 128 ? (NB == 1 ? 3 : 2) : D <= 192 ? 2 : 1; }

  // 32-byte pieces of an LDS row: D/16; XOR swizzle spreads 16 rows over
  // banks (within aligned groups of 8 or 4 pieces, so every piece stays in
  // its row; none where D/16 is not a multiple of 4).
  __device__ static __forceinline__ int swz(int t) {
    return D % 128 == 0 ? (t & 7) : D % 64 == 0 ? ((t >> 1) & 3) : 0;
  }

  __device__ static __forceinline__ void load_q(const half_t* row, bool valid, int g, qreg_t (&q)[kQRegs]) {
#pragma unroll
    for (int s = 0; s < kQRegs; s++) {
      q[s] = valid ? *reinterpret_cast<const half8*>(row + 8 * g + 32 * s) : half8{};
    }
  }

  __device__ static __forceinline__ void load_k(const half_t* slab, int l, kreg_t (&k)[kLoads]) {
    const half_t* row = slab + (l & 15) * D + 8 * (l >> 4);
#pragma unroll
    for (int s = 0; s < kLoads; s++) k[s] = *reinterpret_cast<const half8*>(row + 32 * s);
  }

  __device__ static __forceinline__ void load_v(const half_t* slab, int l, vreg_t (&v)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; u++) {
      const int ci = l + 64 * u; // 16-byte chunk of the 16 x D slab
      v[u] = *reinterpret_cast<const half8*>(slab + 8 * ci);
    }
  }

  // Pages that do not hold whole 16-token chunks: the same loads through a
  // pointer to each token row (K: the lane's row is l & 15; V: load u reads
  // token row v_row(l, u) at column v_col(l, u)).
  __device__ static __forceinline__ void load_k_row(const half_t* row, int l, kreg_t (&k)[kLoads]) {
#pragma unroll
    for (int s = 0; s < kLoads; s++) k[s] = *reinterpret_cast<const half8*>(row + 8 * (l >> 4) + 32 * s);
  }
  __device__ static __forceinline__ int v_row(int l, int u) { return (l + 64 * u) / (D / 8); }
  __device__ static __forceinline__ int v_col(int l, int u) { return 8 * ((l + 64 * u) % (D / 8)); }
  __device__ static __forceinline__ vreg_t load_v_row(const half_t* row, int l, int u) {
    return *reinterpret_cast<const half8*>(row + v_col(l, u));
  }

  __device__ static __forceinline__ void stage_v(half_t* lds, int l, int tok_valid, const vreg_t (&v)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; u++) {
      const int ci = l + 64 * u;
      const int t = ci / (D / 8), c = ci % (D / 8);
      const int piece = (c >> 1) ^ swz(t);
      // Slots past the sequence end may hold anything (unwritten pages);
      // zero them so 0-weight * garbage cannot produce NaN.
      half8 val = t < tok_valid ? v[u] : half8{};
      *reinterpret_cast<half8*>(lds + t * D + piece * 16 + (c & 1) * 8) = val;
    }
  }

  __device__ static __forceinline__ float4v qk(const kreg_t (&k)[kLoads], const qreg_t (&q)[kQRegs]) {
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kLoads; s++) acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(k[s], q[s], acc, 0, 0, 0);
    return acc;
  }

  template <int NB>
  __device__ static __forceinline__ void pv(half_t* lds, int l, const float (&p)[NB][4], float4v (&o)[NB][D / 16]) {
    half4 pb[NB];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) pb[nb] = half4{(half_t)p[nb][0], (half_t)p[nb][1], (half_t)p[nb][2], (half_t)p[nb][3]};
    const int g = l >> 4, qd = l & 15;
    const int row = 4 * g + (qd >> 2);
    const int sw = swz(row);
#pragma unroll
    for (int n = 0; n < D / 16; n++) {
      half_t* addr = lds + row * D + ((n ^ sw) * 16) + 4 * (qd & 3);
      short4v raw = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(addr));
      half4 vt = __builtin_bit_cast(half4, raw);
#pragma unroll
      for (int nb = 0; nb < NB; nb++) o[nb][n] = __builtin_amdgcn_mfma_f32_16x16x16f16(vt, pb[nb], o[nb][n], 0, 0, 0);
    }
  }

  __device__ static __forceinline__ void store_out(half_t* dst, float4v v) {
    half4 h = {(half_t)v[0], (half_t)v[1], (half_t)v[2], (half_t)v[3]};
    *reinterpret_cast<half4*>(dst) = h;
  }
};

template <int D>
struct F32Traits {
  typedef float elem;
  static constexpr int kLoads = D / 16; // 16-byte loads per lane per chunk
  static constexpr int kQRegs = D / 16;
  typedef float4v kreg_t;
  typedef float4v vreg_t;
  typedef float4v qreg_t;

  template <int NB>
  static constexpr int min_blocks() {
    return D == 128 ? (NB == 1 ? 2 : 1) : D <= 64 ? (NB == 1 ? 3 : 2) : D <= 128 ? 2 : 1;
  }

  // 64-byte pieces (16 floats) of an LDS row; rows 4g+j of the four lane
  // groups land in four different pieces (none where D/16 is not a multiple
  // of 4, so that every piece stays in its row).
  __device__ static __forceinline__ int swz(int t) { return (D / 16) % 4 == 0 ? ((t >> 2) & 3) : 0; }

  __device__ static __forceinline__ void load_q(const float* row, bool valid, int g, qreg_t (&q)[kQRegs]) {
#pragma unroll
    for (int u = 0; u < kQRegs; u++) {
      q[u] = valid ? *reinterpret_cast<const float4v*>(row + 16 * u + 4 * g) : float4v{0.f, 0.f, 0.f, 0.f};
    }
  }

  __device__ static __forceinline__ void load_k(const float* slab, int l, kreg_t (&k)[kLoads]) {
    const float* row = slab + (l & 15) * D + 4 * (l >> 4);
#pragma unroll
    for (int u = 0; u < kLoads; u++) k[u] = *reinterpret_cast<const float4v*>(row + 16 * u);
  }

  __device__ static __forceinline__ void load_v(const float* slab, int l, vreg_t (&v)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; u++) v[u] = *reinterpret_cast<const float4v*>(slab + 4 * (l + 64 * u));
  }

  __device__ static __forceinline__ void load_k_row(const float* row, int l, kreg_t (&k)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; u++) k[u] = *reinterpret_cast<const float4v*>(row + 4 * (l >> 4) + 16 * u);
  }
  __device__ static __forceinline__ int v_row(int l, int u) { return (l + 64 * u) / (D / 4); }
  __device__ static __forceinline__ int v_col(int l, int u) { return 4 * ((l + 64 * u) % (D / 4)); }
  __device__ static __forceinline__ vreg_t load_v_row(const float* row, int l, int u) {
    return *reinterpret_cast<const float4v*>(row + v_col(l, u));
  }

  __device__ static __forceinline__ void stage_v(float* lds, int l, int tok_valid, const vreg_t (&v)[kLoads]) {
#pragma unroll
    for (int u = 0; u < kLoads; u++) {
      const int ci = l + 64 * u;
      const int t = ci / (D / 4), c = ci % (D / 4);
      const int piece = (c >> 2) ^ swz(t);
      float4v val = t < tok_valid ? v[u] : float4v{0.f, 0.f, 0.f, 0.f};
      *reinterpret_cast<float4v*>(lds + t * D + piece * 16 + (c & 3) * 4) = val;
    }
  }

  __device__ static __forceinline__ float4v qk(const kreg_t (&k)[kLoads], const qreg_t (&q)[kQRegs]) {
    float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kLoads; u++) {
#pragma unroll
      for (int e = 0; e < 4; e++) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(k[u][e], q[u][e], acc, 0, 0, 0);
    }
    return acc;
  }

  template <int NB>
  __device__ static __forceinline__ void pv(float* lds, int l, const float (&p)[NB][4], float4v (&o)[NB][D / 16]) {
    const int g = l >> 4, qd = l & 15;
#pragma unroll
    for (int n = 0; n < D / 16; n++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int row = 4 * g + j;
        const float vt = lds[row * D + ((n ^ swz(row)) * 16) + qd];
#pragma unroll
        for (int nb = 0; nb < NB; nb++) o[nb][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(vt, p[nb][j], o[nb][n], 0, 0, 0);
      }
    }
  }

  __device__ static __forceinline__ void store_out(float* dst, float4v v) { *reinterpret_cast<float4v*>(dst) = v; }
};

// ---------------------------------------------------------------------------
// Split-context paged attention: one wavefront per unit.
// ---------------------------------------------------------------------------
// Occupancy floor (blocks per CU = wavefronts per SIMD) per dtype: the
// largest that fits each variant without scratch.
//
// BM (block merge): a block of WPB wavefronts holds the partitions of one
// (sequence, KV head, row tile) instead of one partition of kWavesPerBlock
// KV heads, and merges them through LDS at the end: no fp32 partials in HBM
// and no merge launch (which costs about 8 us of launch gap and kernel time
// whatever its work).  The planner uses it when a uniform batch splits every
// context into more than WPB / 2 and at most WPB partitions, WPB = 4, 8 or
// 16 (the wavefronts of a block then do near-equal work); a partition
// without keys still takes part in the block's barriers.
// DENSE: the dense layout of a ragged batch (dense_unit); a separate instantiation,
// so that the slot == partition kernels compile exactly as without it.
// DEPTH: chunks in flight per wavefront.  3 (deep_pipeline plans: 16-row
// tiles whose K and V chunk take 32 VGPRs per lane) costs 192-208 VGPRs, so two
// wavefronts per SIMD instead of three; that pays on ragged batches of few
// sequences, whose live wavefronts do not fill the device and wait on
// latency (16 sequences of 1.9K..14.8K tokens: 120 -> 106 us), and loses
// where a third wavefront per SIMD had work (128 ragged sequences).
// Block shape of a variant: WPB wavefronts; 16-wavefront blocks (4 per SIMD)
// leave 128 VGPRs per lane.  Blocks of 1, 2 or 4 wavefronts without block
// merge compile to the same registers per wavefront.
// Token pages: block-table entries a 16-token chunk can touch when pages
// hold P >= 2 tokens (ceil(15 / P) + 1).
constexpr int kTpWindow = 9;

template <typename Tr, int NB, int DEPTH, int WPB>
constexpr int kernel_min_blocks() {
  return WPB > kWavesPerBlock ? 1 : (DEPTH == 3 ? 2 : Tr::template min_blocks<NB>());
}

template <typename Tr, int D, int NB, bool BM = false, bool DENSE = false, int DEPTH = 2, int WPB = kWavesPerBlock,
          bool TP = false>
__global__ __launch_bounds__(kWaveSize* WPB, (kernel_min_blocks<Tr, NB, DEPTH, WPB>())) void
    paged_attention_kernel(PagedAttentionParams p) {
  typedef typename Tr::elem T;
  constexpr int kTileRows = 16 * NB;
  static_assert(DEPTH == 2 || (DEPTH == 3 && NB == 1 && D * sizeof(T) <= 256 && !BM), "unsupported pipeline depth");
  static_assert(BM ? (WPB == 4 || WPB == 8 || WPB == 16) : (WPB == 1 || WPB == 2 || WPB == 4),
                "block shape: 4, 8 or 16 wavefronts with block merge, 1, 2 or 4 without");
  // Each wavefront's V tile, and (BM, after the key loop) each wavefront's
  // rows (O, m, l) in the same LDS: rows padded by 4 floats so that the 16
  // rows of a float4 store fall in distinct banks.
  constexpr int kMergeStride = D + 4;
  constexpr size_t kTileBytes = (size_t)WPB * kChunkTokens * D * sizeof(T);
  constexpr size_t kMergeBytes = BM ? (size_t)WPB * kTileRows * (kMergeStride + 2) * sizeof(float) : 0;
  __shared__ __attribute__((aligned(16))) char lds_raw[kTileBytes > kMergeBytes ? kTileBytes : kMergeBytes];
  float* const merge_o = reinterpret_cast<float*>(lds_raw);
  float* const merge_ml = merge_o + WPB * kTileRows * kMergeStride;

  const int l = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
  const int64_t unit = (int64_t)blockIdx.x * WPB + wave;
  if (!BM && unit >= p.num_units) return; // BM grids are exact: no wavefront may skip the block barrier
  T* lds = reinterpret_cast<T*>(lds_raw) + (size_t)wave * kChunkTokens * D;

  // KV head fastest: the wavefronts of one (sequence, partition) read the
  // adjacent per-head slabs of the same pages at about the same time, and
  // the dispatcher deals consecutive blocks to the 8 XCDs round-robin.
  // (Dealing each XCD's blocks partition-major across sequences instead
  // measured slower: 142 vs 110 us on 16 sequences of 1K..16K tokens.)
  // BM: block = (sequence, row tile, KV head) with the KV head fastest, so
  // that with 8 KV heads block % 8 (its XCD) is the KV head for every
  // sequence; wavefront = partition.
  int h, part, rt, b;
  SeqInfo s;
  if constexpr (BM) {
    int64_t tile = blockIdx.x;
    part = wave;
    h = (int)(tile % p.num_kv_heads);
    tile /= p.num_kv_heads;
    rt = (int)(tile % p.row_tiles);
    b = (int)(tile / p.row_tiles);
  } else if constexpr (DENSE) {
    h = (int)(unit % p.num_kv_heads);
    rt = 0;
    // part >= max_parts only if a seq_len exceeds max_seq_len (a broken
    // contract): its partial slot would lie in the next tile, so drop it.
    if (!dense_unit(p, unit / p.num_kv_heads, kTileRows, b, part, s) || part >= p.max_parts) return;
  } else {
    int64_t rest = unit;
    h = (int)(rest % p.num_kv_heads);
    rest /= p.num_kv_heads;
    part = (int)(rest % p.max_parts);
    rest /= p.max_parts;
    rt = (int)(rest % p.row_tiles);
    b = (int)(rest / p.row_tiles);
  }
  // Partials are stored tile-major: slot = tile * max_parts + part.
  const int64_t slot = (((int64_t)b * p.num_kv_heads + h) * p.row_tiles + rt) * p.max_parts + part;

  if constexpr (BM || !DENSE) s = load_seq(p, b);
  const int rows = p.group_size * s.q_len;
  const int n_chunks = tile_chunks(s, p.group_size, rt, kTileRows);
  // The tile's n_parts partitions split its chunks evenly (their lengths differ
  // by at most one chunk and lie in (chunks_per_part / 2, chunks_per_part]
  // when n_parts > 1), instead of n_parts - 1 full partitions and a short
  // remainder: in a ragged batch the full-length units set the critical path
  // while the remainders finish early.  A uniform batch whose context is a
  // multiple of chunks_per_part gets the same boundaries either way.
  const int n_parts = tile_parts(s, n_chunks, p.chunks_per_part);
  const int kb0 = s.key_begin / kChunkTokens;
  const int64_t span = n_chunks > kb0 ? n_chunks - kb0 : 0;
  const int k0 = n_parts > 0 ? kb0 + (int)((int64_t)part * span / n_parts) : kb0;
  if (!BM && (n_chunks == 0 || k0 >= n_chunks)) return;
  // BM: k1 <= k0 for a partition without keys (part >= n_parts)
  const int k1 = n_parts > 0 ? min(kb0 + (int)((int64_t)(part + 1) * span / n_parts), n_chunks) : kb0;
  const int g = l >> 4;

  // Query rows of this lane (one per row block) and their causal limits.
  typename Tr::qreg_t q[NB][Tr::kQRegs];
  int limit[NB];
  bool row_valid[NB];
  int q_head[NB], q_tok[NB];
#pragma unroll
  for (int nb = 0; nb < NB; nb++) {
    const int rho = rt * kTileRows + nb * 16 + (l & 15);
    row_valid[nb] = rho < rows;
    const int r = row_valid[nb] ? rho / s.q_len : 0;
    const int i = row_valid[nb] ? rho % s.q_len : 0;
    q_head[nb] = h * p.group_size + r;
    q_tok[nb] = s.q_start + i;
    limit[nb] = row_valid[nb] ? row_limit(s, i) : s.key_end - 1;
    const T* qrow = static_cast<const T*>(p.q) + (int64_t)q_head[nb] * p.q_stride_head + (int64_t)q_tok[nb] * p.q_stride_token;
    Tr::load_q(qrow, row_valid[nb], g, q[nb]);
  }

  float m[NB], lsum[NB];
  float4v o[NB][D / 16];
#pragma unroll
  for (int nb = 0; nb < NB; nb++) {
    m[nb] = -INFINITY;
    lsum[nb] = 0.f;
#pragma unroll
    for (int n = 0; n < D / 16; n++) o[nb][n] = float4v{0.f, 0.f, 0.f, 0.f};
  }

  const T* kpool = static_cast<const T*>(p.key_pool);
  const T* vpool = static_cast<const T*>(p.value_pool);
  // Block-table reads go through the constant address space with a uniform
  // index, so they become scalar loads: a vector load here would make the
  // next address wait on vmcnt(0), i.e. on every K/V load still in flight.
  const const_i32* bt = (const const_i32*)(p.block_tables) + (int64_t)b * p.block_table_stride;
  const int chunks_per_page = p.page_size / kChunkTokens;

  auto slab_offset = [&](int k) -> int64_t {
    const int page = __builtin_amdgcn_readfirstlane(bt[k / chunks_per_page]);
    const int slot0 = (k % chunks_per_page) * kChunkTokens;
    return (((int64_t)page * p.num_kv_heads + h) * p.page_size + slot0) * D;
  };

  auto process = [&](int k, const typename Tr::kreg_t (&kr)[Tr::kLoads], const typename Tr::vreg_t (&vr)[Tr::kLoads]) {
    const int tok0 = k * kChunkTokens;
    asm volatile("" ::: "memory");
    Tr::stage_v(lds, l, s.key_end - tok0, vr);
    float pr[NB][4];
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      float4v sc = Tr::qk(kr, q[nb]);
      float sv[4];
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int tok = tok0 + 4 * g + i;
        sv[i] = tok <= limit[nb] ? sc[i] * p.scale_log2 : -INFINITY;
        mx = fmaxf(mx, sv[i]);
      }
      mx = wave_max_across_groups(mx);
      const float m_new = fmaxf(m[nb], mx);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2f(m[nb] - m_use);
      float psum = 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pr[nb][i] = exp2f(sv[i] - m_use);
        psum += pr[nb][i];
      }
      lsum[nb] = lsum[nb] * alpha + psum;
      m[nb] = m_new;
#pragma unroll
      for (int n = 0; n < D / 16; n++) o[nb][n] *= alpha;
    }
    // V tile written by this wavefront's own lanes: wait for the LDS writes
    // before the transposed reads of other lanes' rows.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    Tr::template pv<NB>(lds, l, pr, o);
  };

  auto load_chunk = [&](int k, typename Tr::kreg_t (&kr)[Tr::kLoads], typename Tr::vreg_t (&vr)[Tr::kLoads]) {
    if constexpr (TP) {
      // Token pages (TP): page sizes that are not a multiple of 16, at least
      // 2, read in place.  Token t lies in page t / P (a multiply and a
      // shift) at slot t mod P; the chunk's tokens lie in at most
      // ceil(15 / P) + 1 <= kTpWindow consecutive block-table entries, read
      // as scalars, and each lane picks its row's page from them.  Rows past
      // the call's last key read the last key's row (masked, and zeroed in
      // the V stage), so every address lies in a page of the sequence.
      const int tok0 = k * kChunkTokens;
      const int tmax = s.key_end - 1; // >= tok0: chunk k holds a key
      auto pdiv = [&](int t) { return (int)(((uint64_t)(uint32_t)t * p.page_magic) >> p.page_magic_shift); };
      const int pf = pdiv(tok0);
      const int pl = pdiv(min(tok0 + kChunkTokens - 1, tmax));
      // Row r's element offset in the pools: (page * Hkv + h) * P + slot,
      // times D, as page * (Hkv P D), one 32 x 32 -> 64-bit product, plus
      // (h P + slot) D in 32 bits (a page of all KV heads holds fewer than
      // 2^31 elements, checked on the host).
      const uint32_t page_elems = (uint32_t)(p.num_kv_heads * p.page_size) * D;
      const uint32_t head_elems = (uint32_t)(h * p.page_size);
      uint32_t roff[1 + Tr::kLoads];
      int pj[1 + Tr::kLoads]; // the row's page, counted from the chunk's first
#pragma unroll
      for (int i = 0; i <= Tr::kLoads; i++) {
        const int r = i == 0 ? (l & 15) : Tr::v_row(l, i - 1);
        const int t = min(tok0 + r, tmax);
        const int pi = pdiv(t);
        roff[i] = (head_elems + (uint32_t)(t - pi * p.page_size)) * D; // (h P + slot) D
        pj[i] = pi - pf;
      }
      uint32_t pg[1 + Tr::kLoads];
#pragma unroll
      for (int i = 0; i <= Tr::kLoads; i++) pg[i] = 0;
#pragma unroll
      for (int j = 0; j < kTpWindow; j++) {
        if (j > 0 && pf + j > pl) break; // the chunk's pages end here (wave-uniform)
        const uint32_t page = (uint32_t)__builtin_amdgcn_readfirstlane(bt[min(pf + j, pl)]);
#pragma unroll
        for (int i = 0; i <= Tr::kLoads; i++) pg[i] = pj[i] == j ? page : pg[i];
      }
      Tr::load_k_row(kpool + ((uint64_t)pg[0] * page_elems + roff[0]), l, kr);
#pragma unroll
      for (int u = 0; u < Tr::kLoads; u++)
        vr[u] = Tr::load_v_row(vpool + ((uint64_t)pg[1 + u] * page_elems + roff[1 + u]), l, u);
    } else {
      const int64_t off = slab_offset(k);
      Tr::load_k(kpool + off, l, kr);
      Tr::load_v(vpool + off, l, vr);
    }
  };

  // DEPTH chunks in flight; a tail past k1 reloads chunk k1 - 1 (an L2 hit)
  // rather than branching.
  typename Tr::kreg_t kbuf[DEPTH][Tr::kLoads];
  typename Tr::vreg_t vbuf[DEPTH][Tr::kLoads];
  if (k0 < k1) { // always, except a BM partition without keys (its chunks lie past the table)
#pragma unroll
    for (int i = 0; i < DEPTH; i++) load_chunk(min(k0 + i, k1 - 1), kbuf[i], vbuf[i]);
  }
  for (int k = k0; k < k1; k += DEPTH) {
#pragma unroll
    for (int i = 0; i < DEPTH; i++) {
      if (i == 0 || k + i < k1) {
        process(k + i, kbuf[i], vbuf[i]);
        load_chunk(min(k + i + DEPTH, k1 - 1), kbuf[i], vbuf[i]);
      }
    }
  }

  if constexpr (BM) {
    // Every wavefront's rows into LDS (a partition without keys holds
    // m = -inf, l = 0, O = 0 and lies past n_parts), then each wavefront
    // merges rows wave, wave + WPB, ... with the arithmetic of
    // merge_partitions_kernel (same order, so the same bits).  The rows
    // overlay the V tiles: every wavefront leaves its key loop first.
    __syncthreads();
#pragma unroll
    for (int nb = 0; nb < NB; nb++) {
      const float ltot = wave_sum_across_groups(lsum[nb]);
      const int rr = nb * 16 + (l & 15);
      float* dst = merge_o + (wave * kTileRows + rr) * kMergeStride;
#pragma unroll
      for (int n = 0; n < D / 16; n++) *reinterpret_cast<float4v*>(dst + 16 * n + 4 * g) = o[nb][n];
      if (g == 0) {
        merge_ml[(wave * kTileRows + rr) * 2 + 0] = m[nb];
        merge_ml[(wave * kTileRows + rr) * 2 + 1] = ltot;
      }
    }
    __syncthreads();
    static_assert(WPB == 4 || WPB == 8 || WPB == 16, "the den sum below is a butterfly over WPB lanes");
    constexpr int kPer = D / kWaveSize;
    // At most one partition per wavefront holds a result (seq_len is clamped to
    // max_seq_len, which the plan splits into at most WPB parts).
    const int n_held = min(n_parts, WPB);
    for (int rr = wave; rr < kTileRows; rr += WPB) {
      const int rho = rt * kTileRows + rr;
      if (rho >= rows || n_held == 0) continue;
      float mj[WPB], wl[WPB];
      float mmax = -INFINITY;
#pragma unroll
      for (int j = 0; j < WPB; j++) {
        mj[j] = j < n_held ? merge_ml[(j * kTileRows + rr) * 2] : -INFINITY;
        mmax = fmaxf(mmax, mj[j]);
      }
      const float m_use = mmax == -INFINITY ? 0.f : mmax;
      float w[WPB];
#pragma unroll
      for (int j = 0; j < WPB; j++) {
        w[j] = j < n_held ? __builtin_amdgcn_exp2f(mj[j] - m_use) : 0.f;
        wl[j] = j < n_held ? w[j] * merge_ml[(j * kTileRows + rr) * 2 + 1] : 0.f;
      }
      // merge_partitions_kernel sums lane j's w_j l_j over the wavefront by
      // xor-shuffles at offsets 32, 16, ..., 1; with the partitions in lanes
      // 0..WPB-1 (0 elsewhere) the steps above WPB / 2 add zeros, and the
      // rest is this butterfly (lane 0's value).
#pragma unroll
      for (int off = WPB / 2; off >= 1; off >>= 1) {
        float t[WPB];
#pragma unroll
        for (int j = 0; j < WPB; j++) t[j] = wl[j] + wl[j ^ off];
#pragma unroll
        for (int j = 0; j < WPB; j++) wl[j] = t[j];
      }
      const float den = wl[0];
      float acc[kPer];
#pragma unroll
      for (int e = 0; e < kPer; e++) acc[e] = 0.f;
      for (int j = 0; j < n_held; j++) {
        const float* src = merge_o + (j * kTileRows + rr) * kMergeStride + l * kPer;
#pragma unroll
        for (int e = 0; e < kPer; e++) acc[e] = fmaf(w[j], src[e], acc[e]);
      }
      const int r = rho / s.q_len, i = rho % s.q_len;
      const float inv = 1.f / den;
      const int64_t srow = (int64_t)(h * p.group_size + r) * p.state_tokens + s.q_start + i;
      if (p.state_o) {
#pragma unroll
        for (int e = 0; e < kPer; e++) p.state_o[srow * D + l * kPer + e] = acc[e] * inv;
        if (l == 0) p.state_lse[srow] = m_use + __log2f(den);
        continue;
      }
      T* out = static_cast<T*>(p.out) + (int64_t)(h * p.group_size + r) * p.out_stride_head +
               (int64_t)(s.q_start + i) * p.out_stride_token + l * kPer;
      const PrefixWeights pw = prefix_weights(p, b, srow, m_use + __log2f(den));
      if (pw.has) {
        const float* src = p.prefix_o + srow * D + l * kPer;
#pragma unroll
        for (int e = 0; e < kPer; e++) out[e] = (T)((pw.wa * src[e] + pw.wb * (acc[e] * inv)) * pw.inv);
      } else {
#pragma unroll
        for (int e = 0; e < kPer; e++) out[e] = (T)(acc[e] * inv);
      }
    }
    return;
  }

#pragma unroll
  for (int nb = 0; nb < NB; nb++) {
    const float ltot = wave_sum_across_groups(lsum[nb]);
    if (n_parts == 1) {
      if (row_valid[nb]) {
        const float inv = 1.f / ltot;
        if (p.state_o) {
          const int64_t srow = (int64_t)q_head[nb] * p.state_tokens + q_tok[nb];
          float* dst = p.state_o + srow * D;
#pragma unroll
          for (int n = 0; n < D / 16; n++) *reinterpret_cast<float4v*>(dst + 16 * n + 4 * g) = o[nb][n] * inv;
          if (g == 0) p.state_lse[srow] = m[nb] + __log2f(ltot);
        } else {
          T* dst =
              static_cast<T*>(p.out) + (int64_t)q_head[nb] * p.out_stride_head + (int64_t)q_tok[nb] * p.out_stride_token;
          const int64_t srow = (int64_t)q_head[nb] * p.state_tokens + q_tok[nb];
          const PrefixWeights pw = prefix_weights(p, b, srow, m[nb] + __log2f(ltot));
          if (pw.has) {
            const float* src = p.prefix_o + srow * D;
#pragma unroll
            for (int n = 0; n < D / 16; n++)
              Tr::store_out(dst + 16 * n + 4 * g,
                            (pw.wa * *reinterpret_cast<const float4v*>(src + 16 * n + 4 * g) + pw.wb * (o[nb][n] * inv)) *
                                pw.inv);
          } else {
#pragma unroll
            for (int n = 0; n < D / 16; n++) Tr::store_out(dst + 16 * n + 4 * g, o[nb][n] * inv);
          }
        }
      }
    } else {
      const int64_t prow = slot * kTileRows + nb * 16 + (l & 15);
      if (row_valid[nb]) {
        float* dst = p.partial_o + prow * D;
#pragma unroll
        for (int n = 0; n < D / 16; n++) *reinterpret_cast<float4v*>(dst + 16 * n + 4 * g) = o[nb][n];
        if (g == 0) {
          p.partial_ml[prow * 2 + 0] = m[nb];
          p.partial_ml[prow * 2 + 1] = ltot;
        }
      }
    }
  }
}

// Merge pass over the partitions of every tile that was split:
//   out = sum_j 2^(m_j - M) o_j / sum_j 2^(m_j - M) l_j,  M = max_j m_j.
// One wavefront per (b, h, rt, row); a 256-thread block covers 4 rows of one
// tile.  Lane j holds partition j's weight (64 partitions per round), the
// partial rows are streamed as one coalesced 4*D-byte row per load with the
// weight broadcast by readlane, eight rows in flight, or (kWide, for plans of
// more than 64 partitions per tile) 32 while at least 32 remain and eight
// after that; always accumulated in partition order, so both give the same
// bits.  The 32-row rounds cost registers: on 8,192 rows of ~32 partitions
// (a cascade suffix pass) they took the merge from 7.9 to 10.1 us.  Rows and tiles that
// were not split exit at once.
// (A fused "last wavefront merges" variant with per-tile arrival counters
// measured 43% slower on MI355X: each wavefront's device-scope release fence
// writes back its XCD's L2, and those write-backs serialise.)
template <typename T, int D, int NB, bool kWide>
__global__ __launch_bounds__(256) void merge_partitions_kernel(PagedAttentionParams p) {
  constexpr int kTileRows = 16 * NB;
  constexpr int kBlocksPerTile = kTileRows / kWavesPerBlock;
  // Output elements per lane: D/64 over the wavefront, or, where D is not a
  // multiple of 64, D/32 over lanes 0..31 (the others hold partition weights
  // only: they re-read lane 31's elements and store nothing).
  constexpr int kPer = D % kWaveSize == 0 ? D / kWaveSize : D / 32;
  constexpr int kDimLanes = D / kPer;
  constexpr int kInFlight = 8;
  constexpr int kInFlightWide = kWide ? 32 : kInFlight;
  const int tile = blockIdx.x / kBlocksPerTile;
  const int lr = (blockIdx.x % kBlocksPerTile) * kWavesPerBlock + __builtin_amdgcn_readfirstlane(threadIdx.x / kWaveSize);
  const int l = lane_id();
  const int ld = kDimLanes == kWaveSize ? l : min(l, kDimLanes - 1); // lane's slice of the row
  const bool stores = kDimLanes == kWaveSize || l < kDimLanes;
  const int rt = tile % p.row_tiles;
  const int h = (tile / p.row_tiles) % p.num_kv_heads;
  const int b = tile / (p.row_tiles * p.num_kv_heads);
  // Partial row of partition j: (tile * max_parts + j) * kTileRows + lr.  The
  // workspace holds max_parts such slots for every tile, so lane j's (m, l)
  // is requested beside the sequence's lengths instead of after them (one
  // round trip less on small calls); slots past the tile's partition count
  // hold nothing of this call and are dropped once that count is known.
  const int64_t prow0 = (int64_t)tile * p.max_parts * kTileRows + lr;
  float2v ml0 = {-INFINITY, 0.f};
  if (l < p.max_parts) ml0 = *reinterpret_cast<const float2v*>(p.partial_ml + (prow0 + (int64_t)l * kTileRows) * 2);
  const SeqInfo s = load_seq(p, b);
  const int rho = rt * kTileRows + lr;
  if (rho >= p.group_size * s.q_len) return;
  const int n_chunks = tile_chunks(s, p.group_size, rt, kTileRows);
  // At most max_parts partials exist per tile (more only if a seq_len exceeds max_seq_len).
  const int n_parts = min(tile_parts(s, n_chunks, p.chunks_per_part), p.max_parts);
  if (n_parts <= 1) return;

  // The first kFirst partial rows need only the partition count: they are in
  // flight while the weights are reduced.  Not in the kWide variant, whose
  // 32-row rounds already keep enough in flight (there the extra registers
  // measured 2% slower on single 32K-token contexts).
  // In groups of 8 rows (one uniform branch per group): a group's rows past
  // the count read the last partial row again (in the tile, an L2 hit) and
  // are left out of the sum below.  (64 / kPer rows, rounded down to whole
  // groups.)
  constexpr int kFirst = kWide ? 0 : 64 / kPer / 8 * 8;
  const float* const base0 = p.partial_o + prow0 * D + ld * kPer;
  float v0[kFirst > 0 ? kFirst : 1][kPer];
#pragma unroll
  for (int g8 = 0; g8 < kFirst; g8 += 8) {
    if (g8 < n_parts) {
#pragma unroll
      for (int u = g8; u < g8 + 8; u++) {
        const int64_t ju = min(u, n_parts - 1);
#pragma unroll
        for (int e = 0; e < kPer; e++) v0[u][e] = base0[ju * kTileRows * D + e];
      }
    }
  }

  float mmax = l < n_parts ? ml0[0] : -INFINITY;
  for (int j = l + kWaveSize; j < n_parts; j += kWaveSize)
    mmax = fmaxf(mmax, p.partial_ml[(prow0 + (int64_t)j * kTileRows) * 2]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, off));
  const float m_use = mmax == -INFINITY ? 0.f : mmax;

  float den = 0.f;
  float acc[kPer];
#pragma unroll
  for (int e = 0; e < kPer; e++) acc[e] = 0.f;
  for (int j0 = 0; j0 < n_parts; j0 += kWaveSize) {
    float w = 0.f;
    if (j0 + l < n_parts) {
      const int64_t prow = prow0 + (int64_t)(j0 + l) * kTileRows;
      const float2v ml = j0 == 0 ? ml0 : *reinterpret_cast<const float2v*>(p.partial_ml + prow * 2);
      w = __builtin_amdgcn_exp2f(ml[0] - m_use); // m = -inf (no visible key) gives 0
      den += w * ml[1];
    }
    const int cnt = min(kWaveSize, n_parts - j0);
    const float* base = p.partial_o + (prow0 + (int64_t)j0 * kTileRows) * D + ld * kPer;
    int jj = 0;
    if (kFirst > 0 && j0 == 0) {
      jj = min(cnt, kFirst);
#pragma unroll
      for (int g8 = 0; g8 < kFirst; g8 += 8) {
        if (g8 < jj) {
#pragma unroll
          for (int u = g8; u < g8 + 8; u++) {
            const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), u));
#pragma unroll
            for (int e = 0; e < kPer; e++) acc[e] = u < jj ? fmaf(wu, v0[u][e], acc[e]) : acc[e];
          }
        }
      }
    }
    // Rows with many partitions (a few long sequences over few KV heads split
    // into hundreds) take 32 partial rows per round trip.
    for (; kWide && jj + kInFlightWide <= cnt; jj += kInFlightWide) {
      float v[kInFlightWide][kPer];
#pragma unroll
      for (int u = 0; u < kInFlightWide; u++)
#pragma unroll
        for (int e = 0; e < kPer; e++) v[u][e] = base[(int64_t)(jj + u) * kTileRows * D + e];
#pragma unroll
      for (int u = 0; u < kInFlightWide; u++) {
        const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), jj + u));
#pragma unroll
        for (int e = 0; e < kPer; e++) acc[e] = fmaf(wu, v[u][e], acc[e]);
      }
    }
    for (; jj + kInFlight <= cnt; jj += kInFlight) {
      float v[kInFlight][kPer];
#pragma unroll
      for (int u = 0; u < kInFlight; u++)
#pragma unroll
        for (int e = 0; e < kPer; e++) v[u][e] = base[(int64_t)(jj + u) * kTileRows * D + e];
#pragma unroll
      for (int u = 0; u < kInFlight; u++) {
        const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), jj + u));
#pragma unroll
        for (int e = 0; e < kPer; e++) acc[e] = fmaf(wu, v[u][e], acc[e]);
      }
    }
    for (; jj < cnt; jj++) {
      const float wu = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), jj));
#pragma unroll
      for (int e = 0; e < kPer; e++) acc[e] = fmaf(wu, base[(int64_t)jj * kTileRows * D + e], acc[e]);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) den += __shfl_xor(den, off);
  const int r = rho / s.q_len, i = rho % s.q_len;
  const float inv = 1.f / den;
  if (p.state_o) {
    const int64_t srow = (int64_t)(h * p.group_size + r) * p.state_tokens + s.q_start + i;
    if (stores) {
#pragma unroll
      for (int e = 0; e < kPer; e++) p.state_o[srow * D + ld * kPer + e] = acc[e] * inv;
    }
    if (l == 0) p.state_lse[srow] = m_use + __log2f(den);
    return;
  }
  T* dst = static_cast<T*>(p.out) + (int64_t)(h * p.group_size + r) * p.out_stride_head +
           (int64_t)(s.q_start + i) * p.out_stride_token + ld * kPer;
  const int64_t srow = (int64_t)(h * p.group_size + r) * p.state_tokens + s.q_start + i;
  const PrefixWeights pw = prefix_weights(p, b, srow, m_use + __log2f(den));
  if (!stores) return;
  if (pw.has) {
    const float* src = p.prefix_o + srow * D + ld * kPer;
#pragma unroll
    for (int e = 0; e < kPer; e++) dst[e] = (T)((pw.wa * src[e] + pw.wb * (acc[e] * inv)) * pw.inv);
    return;
  }
#pragma unroll
  for (int e = 0; e < kPer; e++) dst[e] = (T)(acc[e] * inv);
}

// The split-context kernel without block merge, one unit per wavefront, in
// blocks of WPB wavefronts (its wavefronts share nothing but the block).
template <typename Tr, int D, int NB, int WPB>
hipError_t launch_units(const PagedAttentionPlan& plan, const PagedAttentionParams& params, hipStream_t stream) {
  const int64_t blocks = (plan.num_units + WPB - 1) / WPB;
  if constexpr (!head_dim_all_plans(D)) {
    // The other head dimensions: the plain variant only.
    if (plan.token_pages || plan.dense_parts || plan.deep_pipeline) return hipErrorInvalidValue;
    hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, false, false, 2, WPB>), dim3((unsigned)blocks),
                       dim3(kWaveSize * WPB), 0, stream, params);
    return hipGetLastError();
  } else if (plan.token_pages) {
    // planned with one wavefront per block and two chunks in flight, slot ==
    // partition or the dense layout
    if (WPB != 1 || plan.deep_pipeline) return hipErrorInvalidValue;
    if (plan.dense_parts) {
      if (params.row_tiles != 1) return hipErrorInvalidValue; // dense_unit walks row tile 0 only
      hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, false, true, 2, 1, true>), dim3((unsigned)blocks),
                         dim3(kWaveSize), 0, stream, params);
    } else {
      hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, false, false, 2, 1, true>), dim3((unsigned)blocks),
                         dim3(kWaveSize), 0, stream, params);
    }
  } else if (plan.dense_parts) {
    if (params.row_tiles != 1) return hipErrorInvalidValue; // dense_unit walks row tile 0 only
    hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, false, true, 2, WPB>), dim3((unsigned)blocks),
                       dim3(kWaveSize * WPB), 0, stream, params);
  } else if (plan.deep_pipeline) {
    if constexpr (NB == 1 && D * sizeof(typename Tr::elem) <= 256) {
      hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, false, false, 3, WPB>), dim3((unsigned)blocks),
                         dim3(kWaveSize * WPB), 0, stream, params);
    } else {
      return hipErrorInvalidValue; // planned only where the registers allow three chunks in flight
    }
  } else {
    hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, false, false, 2, WPB>), dim3((unsigned)blocks),
                       dim3(kWaveSize * WPB), 0, stream, params);
  }
  return hipGetLastError();
}

template <typename Tr, int D, int NB>
hipError_t launch_typed(const PagedAttentionPlan& plan, const PagedAttentionParams& params, hipStream_t stream) {
  if (plan.token_pages && !token_page_offsets_fit(params.num_kv_heads, params.page_size, D))
    return hipErrorInvalidValue;
  if constexpr (NB == 1 && head_dim_all_plans(D)) {
    if (plan.block_merge) {
      // One block of block_waves wavefronts per (sequence, KV head, row tile).
      const int64_t tiles = (int64_t)params.num_seqs * params.num_kv_heads * params.row_tiles;
      if (plan.max_parts > plan.block_waves || plan.num_units != tiles * plan.block_waves) return hipErrorInvalidValue;
      if (plan.token_pages) {
        // Token pages: blocks of 4 or 8 wavefronts; not F32 at D=128, whose
        // registers would spill.
        if constexpr (sizeof(typename Tr::elem) == 4 && D == 128) {
          return hipErrorInvalidValue;
        } else if (plan.block_waves == 4) {
          hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, true, false, 2, 4, true>), dim3((unsigned)tiles),
                             dim3(kWaveSize * 4), 0, stream, params);
        } else if (plan.block_waves == 8) {
          hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, true, false, 2, 8, true>), dim3((unsigned)tiles),
                             dim3(kWaveSize * 8), 0, stream, params);
        } else {
          return hipErrorInvalidValue;
        }
      } else if (plan.block_waves == 4) {
        hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, true, false, 2, 4>), dim3((unsigned)tiles),
                           dim3(kWaveSize * 4), 0, stream, params);
      } else if (plan.block_waves == 8) {
        hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, true, false, 2, 8>), dim3((unsigned)tiles),
                           dim3(kWaveSize * 8), 0, stream, params);
      } else if (plan.block_waves == 16) {
        // 16 wavefronts per block leave 128 VGPRs per lane: head_dim 64 only.
        if constexpr (D == 64) {
          hipLaunchKernelGGL((paged_attention_kernel<Tr, D, NB, true, false, 2, 16>), dim3((unsigned)tiles),
                             dim3(kWaveSize * 16), 0, stream, params);
        } else {
          return hipErrorInvalidValue;
        }
      } else {
        return hipErrorInvalidValue;
      }
      return hipGetLastError();
    }
  }
  if (plan.block_merge) return hipErrorInvalidValue; // planned for one 16-row block only
  const int uw = plan.unit_waves == 0 ? kWavesPerBlock : plan.unit_waves;
  hipError_t err;
  if (uw == 1) {
    err = launch_units<Tr, D, NB, 1>(plan, params, stream);
  } else if constexpr (!head_dim_all_plans(D)) {
    return hipErrorInvalidValue; // 1-wavefront blocks only
  } else if (uw == 2) {
    err = launch_units<Tr, D, NB, 2>(plan, params, stream);
  } else if (uw == 4) {
    err = launch_units<Tr, D, NB, 4>(plan, params, stream);
  } else {
    return hipErrorInvalidValue;
  }
  if (err != hipSuccess || plan.max_parts <= 1) return err;
  const int64_t tiles = (int64_t)params.num_seqs * params.num_kv_heads * params.row_tiles;
  if (plan.max_parts > 64) {
    hipLaunchKernelGGL((merge_partitions_kernel<typename Tr::elem, D, NB, true>), dim3((unsigned)(tiles * 4 * NB)),
                       dim3(kWaveSize * kWavesPerBlock), 0, stream, params);
  } else {
    hipLaunchKernelGGL((merge_partitions_kernel<typename Tr::elem, D, NB, false>), dim3((unsigned)(tiles * 4 * NB)),
                       dim3(kWaveSize * kWavesPerBlock), 0, stream, params);
  }
  return hipGetLastError();
}

} // namespace

hipError_t launch_paged_attention(const PagedAttentionPlan& plan, PagedAttentionParams params, hipStream_t stream) {
  params.chunks_per_part = plan.chunks_per_part;
  params.max_parts = plan.max_parts;
  params.row_tiles = plan.row_tiles;
  params.num_units = plan.num_units;
#define MVR_DISPATCH(TR, DD, NBV)                                                             \
  if (plan.head_dim == DD && plan.row_blocks == NBV) return launch_typed<TR<DD>, DD, NBV>(plan, params, stream);
  if (plan.dtype == 1) {
    MVR_DISPATCH(F16Traits, 64, 1)
    MVR_DISPATCH(F16Traits, 64, 2)
    MVR_DISPATCH(F16Traits, 128, 1)
    MVR_DISPATCH(F16Traits, 128, 2)
    MVR_DISPATCH(F16Traits, 32, 1)
    MVR_DISPATCH(F16Traits, 96, 1)
    MVR_DISPATCH(F16Traits, 160, 1)
    MVR_DISPATCH(F16Traits, 192, 1)
    MVR_DISPATCH(F16Traits, 224, 1)
    MVR_DISPATCH(F16Traits, 256, 1)
  } else {
    MVR_DISPATCH(F32Traits, 64, 1)
    MVR_DISPATCH(F32Traits, 64, 2)
    MVR_DISPATCH(F32Traits, 128, 1)
    MVR_DISPATCH(F32Traits, 128, 2)
    MVR_DISPATCH(F32Traits, 32, 1)
    MVR_DISPATCH(F32Traits, 96, 1)
    MVR_DISPATCH(F32Traits, 160, 1)
    MVR_DISPATCH(F32Traits, 192, 1)
    MVR_DISPATCH(F32Traits, 224, 1)
    MVR_DISPATCH(F32Traits, 256, 1)
  }
#undef MVR_DISPATCH
  return hipErrorInvalidValue;
}

namespace {

template <typename Tr, int D, int NB>
int64_t resident_waves_typed() {
  // Cached per device.  Threads driving several devices call this at once:
  // the entries are atomics (relaxed: each is written once with a value that
  // never changes, so racing writers store the same number and a reader sees
  // either 0, and asks the runtime itself, or that number).
  constexpr int kMaxDevices = 64;
  static std::atomic<int64_t> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < kMaxDevices) {
    const int64_t known = cache[dev].load(std::memory_order_relaxed);
    if (known > 0) return known;
  }
  int cus = 0, blocks = 0;
  hipError_t err = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (err == hipSuccess) {
    if constexpr (head_dim_all_plans(D)) {
      err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, paged_attention_kernel<Tr, D, NB>,
                                                         kWaveSize * kWavesPerBlock, 0);
    } else {
      // The variant these head dimensions launch (1-wavefront blocks), in
      // blocks of kWavesPerBlock wavefronts per CU.
      err = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, paged_attention_kernel<Tr, D, NB, false, false, 2, 1>,
                                                         kWaveSize, 0);
      blocks /= kWavesPerBlock;
    }
  }
  if (err != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  // Fill target: at most 2 resident wavefronts per SIMD.  Measured on the
  // batch-64 x 8K decode, 2 per SIMD with longer partitions beat 3 per SIMD
  // with shorter ones (371 vs 395 us): less merge traffic, fewer streams
  // competing for the same DRAM rows.
  const int64_t waves = (int64_t)cus * (blocks < 2 ? blocks : 2) * kWavesPerBlock;
  if (dev < kMaxDevices) cache[dev].store(waves, std::memory_order_relaxed);
  return waves;
}

} // namespace

int64_t paged_attention_resident_waves(int dtype, int head_dim, int row_blocks) {
#define MVR_OCC(TR, DD, NBV) \
  if (head_dim == DD && row_blocks == NBV) return resident_waves_typed<TR<DD>, DD, NBV>();
  if (dtype == 1) {
    MVR_OCC(F16Traits, 64, 1)
    MVR_OCC(F16Traits, 64, 2)
    MVR_OCC(F16Traits, 128, 1)
    MVR_OCC(F16Traits, 128, 2)
    MVR_OCC(F16Traits, 32, 1)
    MVR_OCC(F16Traits, 96, 1)
    MVR_OCC(F16Traits, 160, 1)
    MVR_OCC(F16Traits, 192, 1)
    MVR_OCC(F16Traits, 224, 1)
    MVR_OCC(F16Traits, 256, 1)
  } else {
    MVR_OCC(F32Traits, 64, 1)
    MVR_OCC(F32Traits, 64, 2)
    MVR_OCC(F32Traits, 128, 1)
    MVR_OCC(F32Traits, 128, 2)
    MVR_OCC(F32Traits, 32, 1)
    MVR_OCC(F32Traits, 96, 1)
    MVR_OCC(F32Traits, 160, 1)
    MVR_OCC(F32Traits, 192, 1)
    MVR_OCC(F32Traits, 224, 1)
    MVR_OCC(F32Traits, 256, 1)
  }
#undef MVR_OCC
  return 0;
}

} // namespace mvr
