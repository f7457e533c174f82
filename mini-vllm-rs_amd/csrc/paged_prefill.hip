// Chunked-prefill page-wise attention for gfx950 (F16: MFMA 32x32x16; F32:
// MFMA 32x32x2, see the F32 notes at the products below).
//
// Same contract as paged_attention.hip (common.rs:739-817 semantics: grouped
// rows rho = r*q_len + i, key j visible to query i iff j <= seq_len - q_len + i)
// for requests with many query rows per KV head, where attention is a dense
// contraction (about 950 flop per byte of K/V at q_len 256) and the MFMA
// pipes, not HBM, set the roofline.
//
// Block = G groups of 4 wavefronts over 128 consecutive grouped rows of one
// (sequence, KV head), 32 rows per wavefront.  G = 2: the two groups hold the
// same rows and take alternating key tiles (TT = 64 tokens for F16, 32 for
// F32), so every SIMD runs two wavefronts without splitting the keys across
// blocks; at the end group 1 hands its (O, m, l) to group 0 through LDS and
// group 0 merges and writes.  G = 1 (large F16 grids, two blocks per CU; rows
// of more than 128 elements, one wavefront per SIMD): one group steps through
// every key tile.  Each step stages G TT tokens (one tile per group) in LDS
// through a ring of kStages stages filled by direct-to-LDS loads (32 KiB of K
// and of V per stage at D=128 F16, G = 2):
//   * K tile: 16-byte chunks, XOR swizzle (chunk ^ row%16), read back with
//     ds_read_b128 in the v_mfma_f32_32x32x16_f16 A-operand layout
//     (lane l: token l%32, dims 8*(l/32)+16s);  S^T = K Q^T in D/16 MFMAs
//     per 32 tokens of the tile;
//   * S^T lands with lane l owning row l%32 and 16 tokens per 32; the online softmax
//     is exp2-based with a lazy rescale: the running max only moves (and O is
//     only rescaled) when a score exceeds it by more than 2^8;
//   * V tile: 32-byte-piece swizzle, ds_read_b64_tr_b16 twice per operand
//     gives V^T in the A-operand layout; P^T (fp16) is the B operand straight
//     from the S^T registers;  O^T += V^T P^T in D/16 MFMAs.
// Blocks of one (sequence, KV head) are mapped onto one XCD (workgroups are
// dispatched round-robin over the 8 XCDs), so their shared K/V stays in that
// XCD's L2.  The key range can be split (kv_splits) to fill the device; split
// results go to an fp32 partial workspace that prefill_merge_kernel combines.
#include "paged_prefill.hpp"

#include <math.h>

#include <type_traits>

namespace mvr {
namespace {

typedef _Float16 half_t;
typedef half_t half8 __attribute__((ext_vector_type(8)));
typedef half_t half4 __attribute__((ext_vector_type(4)));
typedef short short4v __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(4))) int32_t const_i32;

constexpr int kRowsPerWave = 32;
constexpr int kRowWaves = 4;                        // wavefronts per 128-row group
constexpr int kBlockRows = kRowsPerWave * kRowWaves;
// Groups of kRowWaves wavefronts per block, taking alternating key tiles
// (PrefillParams::groups, chosen by the host): 2 (two wavefronts per SIMD
// behind one barrier), or 1 (blocks of 4 wavefronts, two per CU up to D=128;
// for rows of more than 128 elements always, whose state, O alone D/2
// registers per lane, needs the up to 512 registers of one wavefront per
// SIMD).
constexpr int kMergeWaves = 4; // wavefronts per block of prefill_merge_kernel
constexpr int kXcds = 8;
#ifndef MVR_PREFILL_STAGES
#define MVR_PREFILL_STAGES 2
#endif
// LDS stages of one key tile per group (2, 3 or 4; the unrolled loop names each
// statically).  Measured on the Qwen2-7B prefill chunk: 2, 3 and 4 stages
// within 1%: the step's loads land under the step's compute.
constexpr int kStages = MVR_PREFILL_STAGES;
static_assert(kStages >= 2 && kStages <= 4, "2, 3 or 4 LDS stages");
constexpr float kRescaleThreshold = 8.0f; // log2 units: p <= 2^8 between rescales

struct SeqRows {
  int seq_len, q_start, q_len, key_end; // keys [0, key_end) belong to this call
};

// 16 bytes per lane from one KV page straight into LDS at lds + 16 * lane
// (buffer_load_dwordx4 ... lds).  The page's base address is wave-uniform
// (a buffer resource in scalar registers) and each lane adds its byte offset
// within the page, which the resource bounds to the page.  The buffer form,
// not global_load_lds: the compiler counts a FLAT-encoded LDS load as a
// possible out-of-order LDS access too, and then waits for every LDS read in
// flight (lgkmcnt(0)) wherever one result is needed, which stalls the MFMAs
// on fragments read ahead of them.  A plain __device__ function: lambdas in
// kernels are also compiled for the host, where these builtins do not exist.
__device__ __forceinline__ void load_page_to_lds16(const void* page, uint32_t page_bytes, uint32_t byte_offset,
                                                   void* lds) {
  // Raw buffer (stride 0), dword 3 = 0x00020000: 32-bit data format, the
  // usual CDNA setting for untyped buffer loads.
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(page), (short)0,
                                                                       (int)page_bytes, 0x00020000);
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)lds, 16, byte_offset, 0, 0, 0);
}

// Tile barrier: waits until at most kNewer of this wavefront's direct-to-LDS
// tile loads are in flight and its LDS reads have returned, then meets the
// other wavefronts.  (__syncthreads() would wait for every load, vmcnt(0),
// and drain the prefetch.)  The wait is the compiler's own s_waitcnt, so its
// bookkeeping of the direct-to-LDS loads stays exact; the empty asm
// statements keep memory accesses from moving across the barrier without
// any further wait.
template <int kNewer>
__device__ __forceinline__ void tile_barrier() {
  __builtin_amdgcn_s_waitcnt((kNewer & 0xF) | ((kNewer >> 4) << 14) | (0x7 << 4)); // vmcnt(n) expcnt(7) lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ SeqRows load_rows(const PrefillParams& p, int b) {
  SeqRows s;
  // single_seq_len is the call's max_seq_len (its pages fit a block-table row,
  // checked on the host): a larger device seq_len is clamped to it.
  s.seq_len = p.seq_lens ? min(p.seq_lens[b], p.single_seq_len) : p.single_seq_len;
  if (p.cu_q_lens) {
    s.q_start = p.cu_q_lens[b];
    s.q_len = p.cu_q_lens[b + 1] - s.q_start;
  } else {
    s.q_start = 0;
    s.q_len = p.single_q_len;
  }
  // Another launch's sequence: no rows here (its blocks exit at once).
  if (s.q_len <= p.skip_q_max && b >= p.skip_seq_lo && b <= p.skip_seq_hi) s.q_len = 0;
  if (p.key_end) { // cascade prefix pass: every row sees every key before key_end
    s.key_end = p.key_end[b];
    s.seq_len = s.key_end + s.q_len;
  } else {
    s.key_end = s.seq_len;
  }
  return s;
}

// Causal limit of query i within this call's keys (common.rs:948-965).
__device__ __forceinline__ int row_limit(const SeqRows& s, int i) { return min(s.seq_len - s.q_len + i, s.key_end - 1); }

// Key tiles of TT tokens the block's rows can see: up to the largest causal
// limit among them.
template <int TT>
__device__ __forceinline__ int block_key_tiles(const SeqRows& s, int group_size, int rt) {
  const int rows = group_size * s.q_len;
  const int rho0 = rt * kBlockRows;
  if (rho0 >= rows || s.q_len <= 0) return 0;
  const int rho1 = min(rho0 + kBlockRows, rows) - 1;
  const int max_i = (rho1 / s.q_len != rho0 / s.q_len) ? s.q_len - 1 : rho1 % s.q_len;
  const int last_key = row_limit(s, max_i); // -1: no key (a prefix pass over an empty prefix)
  return last_key < 0 ? 0 : last_key / TT + 1;
}

template <int D, typename T, int TT, int G>
struct Tile {
  static constexpr int kSuperTokens = TT * G; // tokens per LDS stage: one tile per group
  static constexpr bool kF32 = sizeof(T) == 4;
  static constexpr int kChunkElems = 16 / (int)sizeof(T);            // elements per 16-byte chunk
  static constexpr int kChunksPerRow = D / kChunkElems;              // 16-byte chunks per token row
  static constexpr int kChunks = kSuperTokens * kChunksPerRow;       // per K (or V) stage
  static constexpr int kChunksPerThread = kChunks / (kRowWaves * G * 64); // D/32 (F16 and F32)
  static constexpr int kElems = kSuperTokens * D;
  // V: 32-byte pieces per row, XOR-swizzled with the row.  A transposed read
  // is served per half-wavefront: 4 rows x 2 adjacent pieces, which must land
  // in 8 distinct 32-byte bank groups; 2*(row&3) (D=128) spreads the 4 piece
  // pairs apart, measured conflict-free on gfx950 (row&7 cost 2 extra
  // cycles per read).  At D=64 two rows share a 256-byte bank line and
  // row&3 is already conflict-free.
  // F32 V rows are not swizzled: each half-wavefront reads one whole token row.
  // Other head dimensions keep the XOR inside an aligned group of 4 (D a
  // multiple of 64) or 2 pieces, so that every piece stays in its row.
  __device__ static __forceinline__ int vswz(int t) {
    return kF32 ? 0 : D % 128 == 0 ? 2 * (t & 3) : D % 64 == 0 ? (t & 3) : (t & 1);
  }
  // K: the 16 lanes of a ds_read_b128 pass read one chunk of 16 different
  // rows; XOR with row%16 spreads them over all banks.  Only the low four
  // chunk bits are swizzled, so at F32 D=128 the upper 16 chunks of a row
  // are an immediate offset from the lower ones.  Rows whose
  // chunk count is not a power of two swizzle inside aligned groups of its
  // largest power-of-two factor, so that every chunk stays in its row.
  static constexpr int kSwzGroup = (kChunksPerRow & -kChunksPerRow) < 16 ? (kChunksPerRow & -kChunksPerRow) : 16;
  __device__ static __forceinline__ int kswz(int t) { return t & (kSwzGroup - 1); }
};

// One (sequence, kv head, 128-row tile, key split): each step stages one
// key tile per group, then QK^T, softmax and PV in turn.
template <int D, typename T, int TT, int G, bool TP>
__device__ __forceinline__ void prefill_tile_serial(const PrefillParams& p, const SeqRows& s, int b, int h, int rt,
                                                    int split, int kv_splits) {
  static_assert(G == 1 || G == 2, "one or two wavefront groups");
  typedef Tile<D, T, TT, G> TL;
  constexpr bool kF32 = TL::kF32;
  // Key tile of one group per step: TT tokens = kSub S^T blocks of 32 tokens.
  constexpr int kTileTokens = TT;
  constexpr int kSub = TT / 32;
  static_assert(TT == 32 || (TT == 64 && !kF32), "32-token tiles, or 64 for F16");
  // Q^T fragments (B operand): f16 half8 per 16 dims (32x32x16), f32 float4
  // per 8 dims (four 32x32x2 products).
  typedef typename std::conditional<kF32, float4v, half8>::type qfrag_t;
  constexpr int kQFrags = kF32 ? D / 8 : D / 16;
  // One LDS object per stage and operand: the compiler tracks the
  // direct-to-LDS loads per object, so a read of one stage never waits for
  // the loads still landing in another.
  __shared__ __attribute__((aligned(16))) T k_lds0[TL::kElems], k_lds1[TL::kElems], k_lds2[TL::kElems],
      k_lds3[TL::kElems];
  __shared__ __attribute__((aligned(16))) T v_lds0[TL::kElems], v_lds1[TL::kElems], v_lds2[TL::kElems],
      v_lds3[TL::kElems];
  // Group 1 hands its (m, l) to group 0 here after the key loop (its O goes
  // through the then idle stages).
  __shared__ float ml_xfer[kRowWaves][2][64];

  const int tid = threadIdx.x;
  const int l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rw = wave % kRowWaves;  // rows rw*32 .. +31 of the block
  const int grp = wave / kRowWaves; // key tiles j0 + G i + grp
  const int hh = l >> 5;            // lane half: 0 or 1

  const int rows = p.group_size * s.q_len;
  const int n_tiles = block_key_tiles<TT>(s, p.group_size, rt);
  if (n_tiles == 0) return; // whole block: uniform return before any barrier
  const int tiles_per_split = (n_tiles + kv_splits - 1) / kv_splits;
  const int j0 = split * tiles_per_split;
  const int j1 = min(j0 + tiles_per_split, n_tiles);
  const int64_t slot =
      (int64_t)(((b - p.seq_lo) * p.num_kv_heads + h) * p.row_tiles + rt) * p.kv_splits + split; // kv_splits > 1

  // This lane's query row.
  const int rho = rt * kBlockRows + rw * kRowsPerWave + (l & 31);
  const bool valid = rho < rows;
  const int r = valid ? rho / s.q_len : 0;
  const int i = valid ? rho % s.q_len : 0;
  const int limit = valid ? row_limit(s, i) : -1;
  // Largest and smallest causal limits among the wave's rows.
  int wave_limit = limit;
  for (int off = 1; off < 64; off <<= 1) wave_limit = max(wave_limit, __shfl_xor(wave_limit, off));
  int wave_min_limit = valid ? limit : INT32_MAX;
  for (int off = 1; off < 64; off <<= 1) wave_min_limit = min(wave_min_limit, __shfl_xor(wave_min_limit, off));

  // Q^T as the B operand: lane l holds Q[rho][16s + 8*hh .. +8] (f16) or
  // Q[rho][8s + 4*hh .. +4] (f32).
  qfrag_t q[kQFrags];
  {
    const T* qrow = static_cast<const T*>(p.q) + (int64_t)(h * p.group_size + r) * p.q_stride_head +
                    (int64_t)(s.q_start + i) * p.q_stride_token;
    constexpr int kFragDims = kF32 ? 8 : 16;
#pragma unroll
    for (int st = 0; st < kQFrags; st++)
      q[st] = valid ? *reinterpret_cast<const qfrag_t*>(qrow + kFragDims * st + (kFragDims / 2) * hh) : qfrag_t{};
  }

  float16v o[D / 32];
#pragma unroll
  for (int n = 0; n < D / 32; n++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[n][e] = 0.f;
  float m = -INFINITY, lsum = 0.f;

  const T* kpool = static_cast<const T*>(p.key_pool);
  const T* vpool = static_cast<const T*>(p.value_pool);
  // Block-table reads use the constant address space with a wave-uniform
  // index, so they are scalar loads and never wait on the K/V loads in flight.
  const const_i32* bt = (const const_i32*)(p.block_tables) + (int64_t)b * p.block_table_stride;

  // Page arithmetic by a multiply and a shift (wave-uniform: scalar
  // instructions once per step); the host routes page sizes that are
  // multiples of 16 to this kernel, and (TP, token pages) other sizes that
  // are a multiple of the tokens one load covers.
  auto page_div = [&](int tok) { return (int)(((uint64_t)(uint32_t)tok * p.page_magic) >> p.page_magic_shift); };
  auto page_mod = [&](int tok) { return tok - page_div(tok) * p.page_size; };

  // A stage holds the G TT tokens of one step: tile j0 + G i + g (group g) in
  // rows g TT .. g TT + TT - 1.  Tokens move straight from HBM/L2 into LDS
  // (buffer_load_dwordx4 ... lds: lane i of a wavefront writes 16 bytes at the
  // wavefront's LDS base + 16 i), so they take no registers and no LDS store
  // instructions.  Wavefront w fills the stage's rows w*R .. w*R+R-1 (R = G TT
  // / (4 G) tokens: 16 for F16, 8 for F32), its load u LDS chunks
  // (w*kChunksPerThread + u)*64 .. +63; LDS chunk P
  // holds token row t = P / (D/8), physical chunk P % (D/8), and the lane
  // fetches the logical 16-byte chunk that the K or V swizzle puts there.  A
  // wavefront's R tokens are consecutive and start at a multiple of R, hence
  // lie in one page (page sizes here are multiples of 16): one
  // scalar block-table load, one page address and one bound per wavefront
  // and step.  That page row goes into the buffer base, so a lane's byte
  // offset within the wavefront's tokens never changes and the loop spends no
  // vector instructions on addresses.  With token pages (TP) each load u
  // covers kLoadTokens whole token rows (head_dim 64 and 128), which lie in
  // one page because the page size is a multiple of kLoadTokens: one
  // block-table load, page address and bound per load and step, and the
  // lane's offset counts from the load's first token.
  constexpr int kWaveTokens = TL::kChunksPerThread * 64 / TL::kChunksPerRow; // R
  constexpr int kLoadTokens = 64 / TL::kChunksPerRow;
  static_assert(!TP || 64 % TL::kChunksPerRow == 0, "token pages need loads of whole token rows");
  const int ld_t0 = wave * kWaveTokens;
  uint32_t off_k[TL::kChunksPerThread], off_v[TL::kChunksPerThread];
#pragma unroll
  for (int u = 0; u < TL::kChunksPerThread; u++) {
    const int P = (wave * TL::kChunksPerThread + u) * 64 + l;
    const int t = P / TL::kChunksPerRow, cs = P % TL::kChunksPerRow;
    const int dt = t - ld_t0;
    const int dl = TP ? dt - u * kLoadTokens : dt; // token row from the buffer's base
    off_k[u] = (uint32_t)(dl * D + TL::kChunkElems * (cs ^ TL::kswz(t))) * sizeof(T);
    off_v[u] = (uint32_t)(dl * D + TL::kChunkElems * (2 * ((cs >> 1) ^ TL::vswz(t)) + (cs & 1))) * sizeof(T);
  }
  // Branch-free: every stage issues the same loads.  A group's buffer ends at
  // the call's last key, so lanes of a group that straddles the end read
  // zeros (bounds-checked buffer loads return 0), and a stage past the end
  // re-reads the group holding the last key.  Those tokens lie past every
  // row's causal limit (the last tile is a diagonal tile for every wavefront
  // that sees it), so their scores are masked to -inf, p = 0, and p * (zero
  // or a real V row) = 0.  A wavefront's block-table entry for a stage is
  // read one step before its loads are issued: a scalar load makes its user
  // wait for lgkmcnt(0), which would also drain every LDS read in flight, so
  // the entries are fetched just before a barrier, where lgkmcnt is drained
  // anyway.
  const int n_steps = (j1 - j0 + G - 1) / G;
  const int i_last = max(n_steps - 1, 0);
  constexpr int kPageLoads = TP ? TL::kChunksPerThread : 1; // block-table entries per wavefront and step
  struct Pages {
    int64_t pg[kPageLoads];
  };
  // First token of load u (of the wavefront's tokens without TP), or the
  // call's last key past the end.
  auto load_token = [&](int si, int u) {
    return min((j0 + G * si) * kTileTokens + ld_t0 + u * kLoadTokens, s.key_end - 1);
  };
  auto fetch_pages = [&](int si) {
    Pages pages;
#pragma unroll
    for (int u = 0; u < kPageLoads; u++) pages.pg[u] = bt[page_div(load_token(si, u))]; // wave-uniform
    return pages;
  };
  auto issue_stage = [&](int si, const Pages& pages, T* kb, T* vb) {
    if constexpr (TP) {
      // Per load, all wave-uniform: its first token, that token's page row,
      // and the bytes from there to the end of the page or of the call's
      // keys.  Byte offsets: one 32 x 32 -> 64-bit product for the page (a
      // page of all KV heads is below 4 GiB, checked on the host), 32 bits
      // within it.
      constexpr uint32_t kRowBytes = D * (uint32_t)sizeof(T);
      const uint32_t page_bytes = (uint32_t)(p.num_kv_heads * p.page_size) * kRowBytes;
      const uint32_t head_bytes = (uint32_t)(h * p.page_size) * kRowBytes;
#pragma unroll
      for (int u = 0; u < TL::kChunksPerThread; u++) {
        const int tc = load_token(si, u);
        const int row0 = page_mod(tc);
        const uint64_t base = (uint64_t)(uint32_t)pages.pg[u] * page_bytes + (head_bytes + (uint32_t)row0 * kRowBytes);
        const uint32_t bytes = (uint32_t)min(p.page_size - row0, s.key_end - tc) * kRowBytes;
        const int dst = (wave * TL::kChunksPerThread + u) * 64 * TL::kChunkElems;
        load_page_to_lds16(reinterpret_cast<const char*>(kpool) + base, bytes, off_k[u], kb + dst);
        load_page_to_lds16(reinterpret_cast<const char*>(vpool) + base, bytes, off_v[u], vb + dst);
      }
    } else {
      // All wave-uniform: the wavefront's first token (the last key past the
      // end), its page row, and the bytes from there to the end of the page or
      // of the call's keys.
      const int tc = min((j0 + G * si) * kTileTokens + ld_t0, s.key_end - 1);
      const int row0 = page_mod(tc);
      const int64_t base = ((pages.pg[0] * p.num_kv_heads + h) * p.page_size + row0) * D;
      const uint32_t bytes = (uint32_t)min(p.page_size - row0, s.key_end - tc) * D * (uint32_t)sizeof(T);
#pragma unroll
      for (int u = 0; u < TL::kChunksPerThread; u++) {
        const int dst = (wave * TL::kChunksPerThread + u) * 64 * TL::kChunkElems;
        load_page_to_lds16(kpool + base, bytes, off_k[u], kb + dst);
        load_page_to_lds16(vpool + base, bytes, off_v[u], vb + dst);
      }
    }
  };
  constexpr int kLoadsPerStage = 2 * TL::kChunksPerThread; // per lane
  T* const k_st[4] = {k_lds0, k_lds1, k_lds2, k_lds3};
  T* const v_st[4] = {v_lds0, v_lds1, v_lds2, v_lds3};
  // O hand-off through the idle stages: part n (16 values per lane) of row
  // wave rw in 1024 floats from float (n * 4 + rw) * 1024 of the stages'
  // concatenation, as float4 [e / 4][lane] (16-byte LDS accesses).
  constexpr int kStageFloats = TL::kElems * (int)sizeof(T) / 4;
  static_assert(G == 1 || (D / 32) * kRowWaves * 1024 <= 4 * kStageFloats, "O hand-off exceeds four stages");
  auto xfer_o = [&](int n) -> float* {
    const int f = (n * kRowWaves + rw) * 1024;
    const int obj = f / kStageFloats;
    T* base = obj == 0 ? k_lds0 : obj == 1 ? k_lds1 : obj == 2 ? v_lds0 : v_lds1;
    return reinterpret_cast<float*>(base) + (f % kStageFloats);
  };

  // Per-lane LDS read offsets within this group's 32 rows of a stage.  K:
  // lane reads token l%32, chunk 2s+hh (f16: 8 dims per chunk, F32: 4; the
  // upper 16 chunks of an F32 D=128 row are +64 elements from the lower 16).
  // V^T (f16): step u reads rows 16u+4hh+rsub and +8, 16 columns at
  // 32n+16*(g16&1)+csub, through the transposing read; rows +8 and +16 keep
  // the same swizzle, so they are immediate offsets.  V (F32): lane reads
  // D/32 consecutive elements (D/32)*(l%32) of row 4hh + 8(e/4) + e%4, all
  // rows an immediate offset from one base.
  const int gbase = grp * kTileTokens * D;
  constexpr int kKReads = kF32 ? D / 8 : D / 16; // K fragment reads per tile
  constexpr int kKOffs = kKReads > 8 ? 8 : kKReads;
  int rk[kKOffs];
  {
    const int t = l & 31;
#pragma unroll
    for (int st = 0; st < kKOffs; st++) rk[st] = gbase + t * D + TL::kChunkElems * ((2 * st + hh) ^ TL::kswz(t));
  }
  int rv[kF32 ? 1 : D / 32];
  if constexpr (kF32) {
    rv[0] = gbase + 4 * hh * D + (D / 32) * (l & 31);
  } else {
    const int g16 = l >> 4, qd = l & 15;
    const int rsub = qd >> 2, csub = 4 * (qd & 3);
#pragma unroll
    for (int n = 0; n < D / 32; n++) {
      const int row_a = 4 * hh + rsub;
      const int col = 32 * n + 16 * (g16 & 1) + csub;
      rv[n] = gbase + row_a * D + ((col >> 4) ^ TL::vswz(row_a)) * 16 + (col & 15);
    }
  }
  // The compiler keeps one address register per (stage, read): 24 per stage
  // at D=128, which two stages afford (a loop-variant copy of the offsets
  // that saves them costs 12 adds per step: 56.7 against 53.8 us).
  const float sl2 = p.scale_log2;

  // Wave-uniform tile predicates: a tile is visible when some row of this
  // wavefront sees its first key, and diagonal when some row does not see
  // its last key (then scores are masked).
  auto visible = [&](int j) { return j < j1 && j * kTileTokens <= wave_limit; };
  auto diagonal = [&](int j) { return j * kTileTokens + kTileTokens - 1 > wave_min_limit; };

  // S^T of this group's tile, K read straight into the A operand: f16 D/16
  // MFMAs 32x32x16; F32 D/2 MFMAs 32x32x2, four per 16-byte K read (product
  // c pairs dims 8s+c and 8s+4+c across the lane halves, as Q^T does).
  // (F16, TT = 64: the tile's two 32-token S^T blocks, their products
  // interleaved so that the two accumulation chains overlap.)
  auto qk = [&](const T* kb, const int (&rkx)[kKOffs], float16v (&acc)[kSub]) {
#pragma unroll
    for (int c = 0; c < kSub; c++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[c][e] = 0.f;
    if constexpr (kF32) {
#pragma unroll
      for (int st = 0; st < kKReads; st++) {
        const float4v kf = *reinterpret_cast<const float4v*>(kb + rkx[st % kKOffs] + (st / kKOffs) * 64);
#pragma unroll
        for (int c = 0; c < 4; c++) acc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[c], q[st][c], acc[0], 0, 0, 0);
      }
    } else {
      // (Past the first 8 reads, rows of more than 128 elements: their
      // chunks from the 17th on, +128 elements.)
#pragma unroll
      for (int st = 0; st < D / 16; st++)
#pragma unroll
        for (int c = 0; c < kSub; c++)
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
              *reinterpret_cast<const half8*>(kb + rkx[st % kKOffs] + (st / kKOffs) * 128 + 32 * c * D), q[st], acc[c],
              0, 0, 0);
    }
  };
  // In block c the lane holds tokens tok0 + 32c + 8*(e/4) + 4*hh + e%4 of row rho.
  auto mask = [&](int j, float16v (&sv)[kSub]) {
#pragma unroll
    for (int c = 0; c < kSub; c++) {
      const int rel = limit - j * kTileTokens - 32 * c - 4 * hh;
#pragma unroll
      for (int e = 0; e < 16; e++) sv[c][e] = 8 * (e >> 2) + (e & 3) <= rel ? sv[c][e] : -INFINITY;
    }
  };
  // Scaled row max (log2 units; scale > 0 keeps the order), both lane halves.
  auto row_max = [&](const float16v (&svs)[kSub]) {
    float mxs = -INFINITY;
#pragma unroll
    for (int c = 0; c < kSub; c++) {
      const float16v& sv = svs[c];
      float a = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
      float bb = fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7]));
      float cc = fmaxf(fmaxf(sv[8], sv[9]), fmaxf(sv[10], sv[11]));
      float d = fmaxf(fmaxf(sv[12], sv[13]), fmaxf(sv[14], sv[15]));
      mxs = c == 0 ? fmaxf(fmaxf(a, bb), fmaxf(cc, d)) : fmaxf(mxs, fmaxf(fmaxf(a, bb), fmaxf(cc, d)));
    }
    const float mx = mxs * sl2;
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    return fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
  };
  // Lazy rescale: the running max only moves (and O is only rescaled) when a
  // score exceeds it by more than 2^8, so P stays <= 2^8 in f16.
  auto advance_max = [&](float mx) {
    const bool grow = mx > m + kRescaleThreshold || (m == -INFINITY && mx != -INFINITY);
    if (__any(grow)) {
      const float m_new = grow ? mx : m;
      const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - m_new);
#pragma unroll
      for (int n = 0; n < D / 32; n++) o[n] *= alpha;
      lsum *= alpha;
      m = m_new;
    }
  };
  // P = 2^(s*scale_log2 - m) in f16 (masked keys give 2^-inf = 0) and its row sum.
  auto exps = [&](const float16v (&sv)[kSub], half8 (&pb)[2 * kSub]) {
    const float neg_m = m == -INFINITY ? 0.f : -m;
    float psum = 0.f;
#pragma unroll
    for (int c = 0; c < kSub; c++)
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const float pe = __builtin_amdgcn_exp2f(fmaf(sv[c][e], sl2, neg_m));
        psum += pe;
        pb[2 * c + (e >> 3)][e & 7] = (half_t)pe;
      }
    lsum += psum;
  };
  // O^T += V^T P^T over the tile's 16-token steps u; step u uses tokens
  // 16u + 4*hh + {0..3} and 16u + 8 + 4*hh + {0..3} (the ones this lane holds).
  auto pv = [&](const T* vb, const int (&rvx)[D / 32], const half8 (&pb)[2 * kSub]) {
#pragma unroll
    for (int n = 0; n < D / 32; n++) {
#pragma unroll
      for (int u = 0; u < 2 * kSub; u++) {
        const short4v ra = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vb + rvx[n] + 16 * D * u));
        const short4v rb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vb + rvx[n] + 16 * D * u + 8 * D));
        const half8 vt = __builtin_bit_cast(half8, __builtin_shufflevector(ra, rb, 0, 1, 2, 3, 4, 5, 6, 7));
        o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vt, pb[u], o[n], 0, 0, 0);
      }
    }
  };
  // F32: P stays in the S^T registers (exponentials in place) and is the B
  // operand as it is: product e pairs tokens 8(e/4) + e%4 and +4, which lane
  // halves 0 and 1 hold in element e.  The A operand is V itself: lane l
  // takes V[token][(D/32)*(l%32) + n] for product n, so O^T block n holds
  // dims (D/32)*i + n (i = its row), one 16- or 8-byte read per token pair.
  auto exps32 = [&](float16v& sv) {
    const float neg_m = m == -INFINITY ? 0.f : -m;
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      sv[e] = __builtin_amdgcn_exp2f(fmaf(sv[e], sl2, neg_m));
      psum += sv[e];
    }
    lsum += psum;
  };
  // A lane's D/32 consecutive elements of a row: one vector access where that
  // is 1, 2 or 4 elements, one access per element otherwise (D = 96).
  constexpr bool kVecRow = D / 32 == 1 || D / 32 == 2 || D / 32 == 4;
  typedef float vrow_t __attribute__((ext_vector_type(kVecRow ? D / 32 : 1)));
  auto pv32 = [&](const T* vb, const float16v& pe) {
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const T* src = vb + rv[0] + (8 * (e >> 2) + (e & 3)) * D;
      if constexpr (kVecRow) {
        const vrow_t vf = *reinterpret_cast<const vrow_t*>(src);
#pragma unroll
        for (int n = 0; n < D / 32; n++) o[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[n], pe[e], o[n], 0, 0, 0);
      } else {
#pragma unroll
        for (int n = 0; n < D / 32; n++) o[n] = __builtin_amdgcn_mfma_f32_32x32x2f32(src[n], pe[e], o[n], 0, 0, 0);
      }
    }
  };

  // Pipeline over steps of two tiles in kStages LDS stages; step i uses stage
  // i % kStages.  Step i issues the loads of step i + kStages - 1 into the
  // stage that held step i - 1 (released by the previous barrier), then each
  // group attends its tile, and the wavefronts meet once step i + 1 has
  // landed.  Loads past the last step re-read it (clamped) into stages nobody
  // reads again.  (Skewing group 1 by half a step, so that its softmax would
  // fall under group 0's MFMAs, measured slower: 58.4 against 55.7 us.)
  constexpr int kAhead = kStages - 1;                       // steps issued ahead of the one consumed
  constexpr int kInFlight = (kStages - 2) * kLoadsPerStage; // loads a barrier leaves in flight
  // Every stage starts zeroed: should an out-of-range lane of a direct-to-LDS
  // load leave its 16 bytes unwritten rather than write the zeros it read,
  // they hold zeros or an earlier tile's keys, never another kernel's data.
  // Each lane clears exactly the bytes its own loads fill, and waits for the
  // stores before issuing them.
#pragma unroll
  for (int a = 0; a < kStages; a++) {
#pragma unroll
    for (int u = 0; u < TL::kChunksPerThread; u++) {
      const int e = ((wave * TL::kChunksPerThread + u) * 64 + l) * TL::kChunkElems;
      *reinterpret_cast<u32x4*>(k_st[a] + e) = u32x4{0u, 0u, 0u, 0u};
      *reinterpret_cast<u32x4*>(v_st[a] + e) = u32x4{0u, 0u, 0u, 0u};
    }
  }
  __builtin_amdgcn_s_waitcnt(0xC07F); // lgkmcnt(0)
#pragma unroll
  for (int a = 0; a < kAhead; a++) issue_stage(min(a, i_last), fetch_pages(min(a, i_last)), k_st[a], v_st[a]);
  Pages next_pages = fetch_pages(min(kAhead, i_last));
  tile_barrier<kInFlight>(); // step 0 landed

  // Steps whose two tiles every row of the block sees in full need neither
  // visibility tests nor masks.
  auto step_clear = [&](int si, auto st_c) {
    constexpr int st = decltype(st_c)::value;
    issue_stage(min(si + kAhead, i_last), next_pages, k_st[(st + kAhead) % kStages], v_st[(st + kAhead) % kStages]);
    float16v sc[kSub];
    qk(k_st[st], rk, sc);
    advance_max(row_max(sc));
    if constexpr (kF32) {
      exps32(sc[0]);
      pv32(v_st[st], sc[0]);
    } else {
      half8 pb[2 * kSub];
      exps(sc, pb);
      pv(v_st[st], rv, pb);
    }
    next_pages = fetch_pages(min(si + kStages, i_last));
    tile_barrier<kInFlight>();
  };
  auto step = [&](int si, auto st_c) {
    constexpr int st = decltype(st_c)::value;
    issue_stage(min(si + kAhead, i_last), next_pages, k_st[(st + kAhead) % kStages], v_st[(st + kAhead) % kStages]);
    const int j = j0 + G * si + grp;
    if (visible(j)) {
      float16v sc[kSub];
      qk(k_st[st], rk, sc);
      if (diagonal(j)) mask(j, sc);
      advance_max(row_max(sc));
      if constexpr (kF32) {
        exps32(sc[0]);
        pv32(v_st[st], sc[0]);
      } else {
        half8 pb[2 * kSub];
        exps(sc, pb);
        pv(v_st[st], rv, pb);
      }
    }
    next_pages = fetch_pages(min(si + kStages, i_last));
    tile_barrier<kInFlight>();
  };
  // Smallest causal limit among the block's valid rows.
  int block_min_limit;
  {
    const int rho0 = rt * kBlockRows;
    const int rho_last = min(rho0 + kBlockRows, rows) - 1;
    const int min_i = rho0 / s.q_len != rho_last / s.q_len ? 0 : rho0 % s.q_len;
    block_min_limit = row_limit(s, min_i);
  }
  const int clear_tiles = min(j1, (block_min_limit + 1) / kTileTokens); // tiles j < this are clear
  // Clear steps (both tiles clear); their count is a multiple of kStages so
  // that the general loop starts on stage 0.
  const int i_mid = max(0, (clear_tiles - j0) / G) / kStages * kStages;

  // Unrolled by kStages so that every stage is named statically: LDS
  // addresses become immediate offsets and each stage is its own object.
#define MVR_STAGE(K) std::integral_constant<int, K>()
  for (int si = 0; si < i_mid; si += kStages) {
    step_clear(si, MVR_STAGE(0));
    step_clear(si + 1, MVR_STAGE(1));
    if constexpr (kStages >= 3) step_clear(si + 2, MVR_STAGE(2));
    if constexpr (kStages == 4) step_clear(si + 3, MVR_STAGE(3));
  }
  for (int si = i_mid; si < n_steps; si += kStages) {
    step(si, MVR_STAGE(0));
    if (si + 1 >= n_steps) break;
    step(si + 1, MVR_STAGE(1));
    if constexpr (kStages >= 3) {
      if (si + 2 >= n_steps) break;
      step(si + 2, MVR_STAGE(2));
    }
    if constexpr (kStages == 4) {
      if (si + 3 >= n_steps) break;
      step(si + 3, MVR_STAGE(3));
    }
  }
#undef MVR_STAGE
  // Every issued load has landed before the LDS is reused or the block exits
  // (the last barrier left up to kStages - 2 steps of clamped re-reads in
  // flight).  Each wavefront waits for its own loads; the barrier then
  // makes sure no wavefront's loads still land in the stages that carry the
  // hand-off below.
  __builtin_amdgcn_s_waitcnt(0x0070); // vmcnt(0) expcnt(7) lgkmcnt(0)
  __syncthreads();

  // Group 1 hands its running state to group 0, which merges:
  //   M = max(m0, m1), o = 2^(m0-M) o0 + 2^(m1-M) o1, l likewise.
  if constexpr (G == 2) {
    if (grp == 1) {
#pragma unroll
      for (int n = 0; n < D / 32; n++) {
        float4v* dst = reinterpret_cast<float4v*>(xfer_o(n));
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++)
          dst[e4 * 64 + l] = float4v{o[n][4 * e4], o[n][4 * e4 + 1], o[n][4 * e4 + 2], o[n][4 * e4 + 3]};
      }
      ml_xfer[rw][0][l] = m;
      ml_xfer[rw][1][l] = lsum;
    }
    __syncthreads();
    if (grp == 1) return;
    {
      const float m1 = ml_xfer[rw][0][l];
      const float l1 = ml_xfer[rw][1][l];
      const float mm = fmaxf(m, m1);
      const float a0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mm);
      const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mm);
#pragma unroll
      for (int n = 0; n < D / 32; n++) {
        const float4v* src = reinterpret_cast<const float4v*>(xfer_o(n));
#pragma unroll
        for (int e4 = 0; e4 < 4; e4++) {
          const float4v x = src[e4 * 64 + l];
#pragma unroll
          for (int c = 0; c < 4; c++) o[n][4 * e4 + c] = a0 * o[n][4 * e4 + c] + a1 * x[c];
        }
      }
      lsum = a0 * lsum + a1 * l1;
      m = mm;
    }
  }

  const float ltot = lsum + __shfl_xor(lsum, 32);
  if constexpr (kF32) {
    // Lane holds O^T[d][rho] for d = (D/32)*(8*(e/4) + 4*hh + e%4) + n.
    auto put = [&](float* dst, float scale) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        float* row = dst + (D / 32) * (8 * (e >> 2) + 4 * hh + (e & 3));
        if constexpr (kVecRow) {
          vrow_t v;
#pragma unroll
          for (int n = 0; n < D / 32; n++) v[n] = o[n][e] * scale;
          *reinterpret_cast<vrow_t*>(row) = v;
        } else {
#pragma unroll
          for (int n = 0; n < D / 32; n++) row[n] = o[n][e] * scale;
        }
      }
    };
    if (!valid) return;
    if (kv_splits > 1) {
      const int64_t prow = slot * kBlockRows + rw * kRowsPerWave + (l & 31);
      put(p.partial_o + prow * D, 1.f);
      if (hh == 0) {
        p.partial_ml[prow * 2 + 0] = m;
        p.partial_ml[prow * 2 + 1] = ltot;
      }
    } else if (p.state_o) {
      const int64_t srow = (int64_t)(h * p.group_size + r) * p.state_tokens + s.q_start + i;
      put(p.state_o + srow * D, 1.f / ltot);
      if (hh == 0) p.state_lse[srow] = m + __log2f(ltot);
    } else {
      put(static_cast<float*>(p.out) + (int64_t)(h * p.group_size + r) * p.out_stride_head +
              (int64_t)(s.q_start + i) * p.out_stride_token,
          1.f / ltot);
    }
    return;
  }
  // Lane holds O^T[d][rho] for d = 32n + 8*(e/4) + 4*hh + e%4.
  if (kv_splits == 1) {
    if (valid && p.state_o) {
      const float inv = 1.f / ltot;
      const int64_t srow = (int64_t)(h * p.group_size + r) * p.state_tokens + s.q_start + i;
      float* dst = p.state_o + srow * D;
#pragma unroll
      for (int n = 0; n < D / 32; n++)
#pragma unroll
        for (int a = 0; a < 4; a++)
          *reinterpret_cast<float4v*>(dst + 32 * n + 8 * a + 4 * hh) =
              float4v{o[n][4 * a], o[n][4 * a + 1], o[n][4 * a + 2], o[n][4 * a + 3]} * inv;
      if (hh == 0) p.state_lse[srow] = m + __log2f(ltot);
    } else if (!p.state_o) {
      // The wavefront's 32 rows go through LDS (its own 32 x D slice of the
      // idle V stage 0: the hand-off used K stages 0 and 1 only), so that the
      // output is written 16 bytes per lane along whole rows.  Written
      // straight from the MFMA layout, each store instruction would touch 32
      // rows 8 bytes at a time: 3.6 of the 47 us of the Qwen2-7B prefill
      // chunk.  The slice swizzles 16-byte chunks with the row (chunk ^ row %
      // chunks), so neither the 8-byte writes nor the 16-byte reads collide
      // in LDS banks.  A wavefront's LDS accesses complete in order, so its
      // reads see its writes.  (Head dimensions whose rows do not tile a
      // wavefront's 64 lanes in whole 16-byte chunks, or whose V stage is
      // too small or carries part of the hand-off, store straight from the
      // MFMA layout.)
      constexpr int kChunksPerRow = D / 8;
      constexpr bool kStaged = 64 % kChunksPerRow == 0 && kRowWaves * kRowsPerWave * D <= TL::kElems &&
                               (D / 32) * kRowWaves * 1024 <= 2 * kStageFloats;
      if constexpr (!kStaged) {
        if (valid) {
          const float inv = 1.f / ltot;
          half_t* dst = static_cast<half_t*>(p.out) + (int64_t)(h * p.group_size + r) * p.out_stride_head +
                        (int64_t)(s.q_start + i) * p.out_stride_token;
#pragma unroll
          for (int n = 0; n < D / 32; n++)
#pragma unroll
            for (int a = 0; a < 4; a++)
              *reinterpret_cast<half4*>(dst + 32 * n + 8 * a + 4 * hh) =
                  half4{(half_t)(o[n][4 * a] * inv), (half_t)(o[n][4 * a + 1] * inv), (half_t)(o[n][4 * a + 2] * inv),
                        (half_t)(o[n][4 * a + 3] * inv)};
        }
      } else {
        half_t* slice = reinterpret_cast<half_t*>(v_lds0) + rw * kRowsPerWave * D;
        const float inv = valid ? 1.f / ltot : 0.f;
        const int row = l & 31;
#pragma unroll
        for (int n = 0; n < D / 32; n++)
#pragma unroll
          for (int a = 0; a < 4; a++) {
            const half4 v4 = {(half_t)(o[n][4 * a] * inv), (half_t)(o[n][4 * a + 1] * inv),
                              (half_t)(o[n][4 * a + 2] * inv), (half_t)(o[n][4 * a + 3] * inv)};
            const int chunk = (4 * n + a) ^ (row & (kChunksPerRow - 1));
            *reinterpret_cast<half4*>(slice + row * D + chunk * 8 + 4 * hh) = v4;
          }
        constexpr int kRowsPerRead = 64 / kChunksPerRow;
        // The lane index is opaque to the optimiser here, so the read offsets
        // below are computed where they are used, not hoisted to the kernel's
        // entry, where (in the catch-up loop) they were spilled to a private
        // segment.
        int le = l;
        asm volatile("" : "+v"(le));
        const int cc = le % kChunksPerRow;
#pragma unroll
        for (int k = 0; k < kRowsPerWave / kRowsPerRead; k++) {
          const int rr = k * kRowsPerRead + le / kChunksPerRow; // row of the wavefront's 32
          const half8 v8 = *reinterpret_cast<const half8*>(slice + rr * D + (cc ^ (rr & (kChunksPerRow - 1))) * 8);
          const int rho_w = rt * kBlockRows + rw * kRowsPerWave + rr;
          if (rho_w < rows) {
            const int rr_r = rho_w / s.q_len, rr_i = rho_w % s.q_len;
            half_t* dst = static_cast<half_t*>(p.out) + (int64_t)(h * p.group_size + rr_r) * p.out_stride_head +
                          (int64_t)(s.q_start + rr_i) * p.out_stride_token;
            *reinterpret_cast<half8*>(dst + cc * 8) = v8;
          }
        }
      }
    }
  } else if (valid) {
    const int64_t prow = slot * kBlockRows + rw * kRowsPerWave + (l & 31);
    float* dst = p.partial_o + prow * D;
#pragma unroll
    for (int n = 0; n < D / 32; n++)
#pragma unroll
      for (int a = 0; a < 4; a++)
        *reinterpret_cast<float4v*>(dst + 32 * n + 8 * a + 4 * hh) =
            float4v{o[n][4 * a], o[n][4 * a + 1], o[n][4 * a + 2], o[n][4 * a + 3]};
    if (hh == 0) {
      // m is kept in log2 units of the scaled score, as the decode partials.
      p.partial_ml[prow * 2 + 0] = m;
      p.partial_ml[prow * 2 + 1] = ltot;
    }
  }
}

// Key tile per group and step: 64 tokens for F16 (the per-tile row max,
// rescale test, barrier and block-table work spread over twice the keys:
// 48.8 -> 47.0 us on the Qwen2-7B chunk, 32.3 -> 31.5 us on a Qwen2-0.5B-shape
// chunk), 32 for F32, whose 64-token stages would not fit in LDS.
template <int D, typename T>
constexpr int prefill_tile_tokens() {
  return sizeof(T) == 4 ? 32 : 64;
}

// Main grid: block x covers (sequence, kv head, row tile, key split) of the
// main range.  XCD-aware decode: block x runs on XCD x % 8 and all blocks of
// one (sequence, kv head) pair sit on the same XCD, so their shared K/V stays
// in that XCD's L2 (with fewer pairs than XCDs, plain linear order keeps
// every XCD busy).  Catch-up blocks follow the main grid.
template <int D, typename T, int G, bool TP>
__device__ __forceinline__ void prefill_tile(const PrefillParams& p, const SeqRows& s, int b, int h, int rt, int split,
                                             int kv_splits) {
  prefill_tile_serial<D, T, prefill_tile_tokens<D, T>(), G, TP>(p, s, b, h, rt, split, kv_splits);
}

__host__ __device__ __forceinline__ int64_t prefill_main_blocks(const PrefillParams& p) {
  const int64_t pairs = (int64_t)(p.seq_count ? p.seq_count : p.num_seqs) * p.num_kv_heads;
  const int64_t per_pair = (int64_t)p.row_tiles * p.kv_splits;
  return pairs >= kXcds ? kXcds * ((pairs + kXcds - 1) / kXcds) * per_pair : pairs * per_pair;
}

// TP: pages that are not a multiple of 16 tokens, read in place (head_dim 64
// and 128; the page size a multiple of the tokens one load covers).
template <int D, typename T, int G, bool TP>
__global__ __launch_bounds__(kRowWaves* G * 64, (G == 1 && D <= 128) ? 2 : 1) void paged_prefill_kernel(PrefillParams p) {
  const int x = blockIdx.x;
  const int main_seqs = p.seq_count ? p.seq_count : p.num_seqs;
  const int main_blocks = (int)prefill_main_blocks(p);
  if (x >= main_blocks) {
    // Catch-up block: every (kv head, row tile) of one sequence, unsplit.
    const int b = p.catch_lo + (x - main_blocks);
    if (b >= p.seq_lo && b < p.seq_lo + main_seqs) return; // the main grid covers it
    const SeqRows s = load_rows(p, b);
    if (s.q_len <= 0) return;
    for (int h = 0; h < p.num_kv_heads; h++)
      for (int rt = 0; rt < p.row_tiles; rt++) {
        prefill_tile<D, T, G, TP>(p, s, b, h, rt, 0, 1);
        __syncthreads(); // group 0's hand-off reads end before the next tile refills the stages
      }
    return;
  }
  const int per_pair = p.row_tiles * p.kv_splits;
  const int pairs = main_seqs * p.num_kv_heads;
  int pair, local;
  if (pairs >= kXcds) {
    const int k_on_xcd = x / kXcds;
    pair = (x % kXcds) + kXcds * (k_on_xcd / per_pair);
    local = k_on_xcd % per_pair;
  } else {
    pair = x / per_pair;
    local = x % per_pair;
  }
  if (pair >= pairs) return;
  const int h = pair % p.num_kv_heads;
  const int b = p.seq_lo + pair / p.num_kv_heads;
  const int split = local % p.kv_splits;
  const SeqRows s = load_rows(p, b);
  // Longest first: a tile's causal key range grows with the query positions
  // of its rows, so the pair's tiles are dispatched in decreasing order of
  // work.  When q_len is a multiple of the tile (rows r*q_len + i, tile j of
  // query head r covers positions 128j .. 128j+127), that is position tile j
  // descending across all query heads of the group, and block indices past
  // the sequence's own tiles keep their index (no rows: they exit);
  // otherwise row tiles in reverse.  Either way a bijection of [0, row_tiles):
  // the same blocks in another order, bit for bit.  Measured on
  // fresh prompts: Llama-3-8B 1 x 2048 F16 75.3 (in order) -> 70.7 (reverse)
  // -> 58.0 us (by position), F32 512.1 -> 480.6 -> 325.9, Qwen2-7B 1 x 8192
  // 667.7 -> 632.6 -> 517.4; chunks on a long prefix level.
  int rt;
  {
    const int idx = local / p.kv_splits;
    const int tq = s.q_len / kBlockRows; // tiles per query head
    if (s.q_len > 0 && s.q_len % kBlockRows == 0) {
      rt = idx < p.group_size * tq ? (idx % p.group_size) * tq + (tq - 1 - idx / p.group_size) : idx;
    } else {
      rt = p.row_tiles - 1 - idx;
    }
  }
  prefill_tile<D, T, G, TP>(p, s, b, h, rt, split, p.kv_splits);
}

// Merges the kv_splits partial results of every block tile:
//   out = sum_j 2^(m_j - M) o_j / sum_j 2^(m_j - M) l_j.
// One wavefront per merge_rows<D>() output rows of a tile (a 256-thread
// block covers 4 x that many rows): lane j holds split j's weight, broadcast
// by readlane.  Every split slot's (m, l) and partial row for all of the
// wavefront's rows are loaded at once, before the rows' bounds are known
// (the slots exist for all kv_splits <= kMaxSplits; those of splits that did
// not run are loaded and never used), so the wavefront costs one round trip.
// Empty splits (no visible key) hold m = -inf, l = 0 and weigh nothing.
constexpr int kMaxSplits = 8; // the planner's cap on kv_splits
// Output rows per wavefront.  Measured on key-split prefill calls: at D=64 (one
// element per lane) two rows per wavefront took a Qwen2-0.5B-shape chunk from
// 34.5 to 32.5 us; at D=128 two or four rows slowed the shared-prompt
// cascade's prefix pass by 1-4 us, so it keeps one.
template <int D>
constexpr int merge_rows() {
  return D == 64 ? 2 : 1;
}
template <int D, typename T, int TT>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p) {
  // Output elements per lane: D/64 over the wavefront, or, where D is not a
  // multiple of 64, D/32 over lanes 0..31 (the others hold split weights
  // only: they re-read lane 31's elements and store nothing).
  constexpr int kPer = D % 64 == 0 ? D / 64 : D / 32;
  constexpr int kDimLanes = D / kPer;
  constexpr int kMergeRows = merge_rows<D>();
  constexpr int kBlocksPerTile = kBlockRows / (kMergeWaves * kMergeRows);
  const int tile = blockIdx.x / kBlocksPerTile; // (b - seq_lo, h, rt)
  const int lr0 = ((blockIdx.x % kBlocksPerTile) * kMergeWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)) *
                  kMergeRows;
  const int l = threadIdx.x & 63;
  const int ld = kDimLanes == 64 ? l : min(l, kDimLanes - 1); // lane's slice of the row
  const int rt = tile % p.row_tiles;
  const int h = (tile / p.row_tiles) % p.num_kv_heads;
  const int b = p.seq_lo + tile / (p.row_tiles * p.num_kv_heads);
  const int splits = min(p.kv_splits, kMaxSplits);
  const int64_t prow0 = (int64_t)tile * p.kv_splits * kBlockRows + lr0; // split j, row r: prow0 + j * kBlockRows + r
  float mj_raw[kMergeRows], lj_raw[kMergeRows], v[kMergeRows][kMaxSplits][kPer];
#pragma unroll
  for (int r = 0; r < kMergeRows; r++) {
    const int64_t pr = prow0 + (int64_t)l * kBlockRows + r;
    mj_raw[r] = l < splits ? p.partial_ml[pr * 2] : -INFINITY;
    lj_raw[r] = l < splits ? p.partial_ml[pr * 2 + 1] : 0.f;
#pragma unroll
    for (int j = 0; j < kMaxSplits; j++) {
      const float* src = p.partial_o + (prow0 + (int64_t)j * kBlockRows + r) * D + ld * kPer;
#pragma unroll
      for (int e = 0; e < kPer; e++) v[r][j][e] = j < splits ? src[e] : 0.f;
    }
  }
  const SeqRows s = load_rows(p, b);
  const int rows = p.group_size * s.q_len;
  const int n_tiles = block_key_tiles<TT>(s, p.group_size, rt);
  if (n_tiles == 0) return;
  const int tiles_per_split = (n_tiles + p.kv_splits - 1) / p.kv_splits;
  const int n_parts = min((n_tiles + tiles_per_split - 1) / tiles_per_split, splits); // splits that ran
#pragma unroll
  for (int r = 0; r < kMergeRows; r++) {
    const int rho = rt * kBlockRows + lr0 + r;
    if (rho >= rows) break;
    const float mj = l < n_parts ? mj_raw[r] : -INFINITY;
    float mmax = mj;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, off));
    const float m_use = mmax == -INFINITY ? 0.f : mmax;
    const float w = mj == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mj - m_use);
    float den = l < n_parts ? w * lj_raw[r] : 0.f;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) den += __shfl_xor(den, off);
    float acc[kPer];
#pragma unroll
    for (int e = 0; e < kPer; e++) acc[e] = 0.f;
#pragma unroll
    for (int j = 0; j < kMaxSplits; j++) {
      if (j < n_parts) {
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
#pragma unroll
        for (int e = 0; e < kPer; e++) acc[e] = fmaf(wj, v[r][j][e], acc[e]);
      }
    }
    const int qr = rho / s.q_len, i = rho % s.q_len;
    const float inv = 1.f / den;
    if (p.state_o) {
      const int64_t srow = (int64_t)(h * p.group_size + qr) * p.state_tokens + s.q_start + i;
      if (kDimLanes == 64 || l < kDimLanes) {
#pragma unroll
        for (int e = 0; e < kPer; e++) p.state_o[srow * D + ld * kPer + e] = acc[e] * inv;
      }
      if (l == 0) p.state_lse[srow] = m_use + __log2f(den);
      continue;
    }
    if (kDimLanes < 64 && l >= kDimLanes) continue;
    T* dst = static_cast<T*>(p.out) + (int64_t)(h * p.group_size + qr) * p.out_stride_head +
             (int64_t)(s.q_start + i) * p.out_stride_token + ld * kPer;
#pragma unroll
    for (int e = 0; e < kPer; e++) dst[e] = (T)(acc[e] * inv);
  }
}

template <int D, typename T>
hipError_t launch_typed(const PrefillParams& params, hipStream_t stream) {
  constexpr int TT = prefill_tile_tokens<D, T>();
  const int64_t blocks = prefill_main_blocks(params) + params.catch_count;
  if (params.page_size % 16 != 0) {
    if (!prefill_token_pages_supported(params.page_size, params.num_kv_heads, D, (int)sizeof(T)))
      return hipErrorInvalidValue;
    if constexpr (D == 64 || D == 128) {
      if (params.groups == 1)
        hipLaunchKernelGGL((paged_prefill_kernel<D, T, 1, true>), dim3((unsigned)blocks), dim3(kRowWaves * 64),
                           0, stream, params);
      else if (params.groups == 2)
        hipLaunchKernelGGL((paged_prefill_kernel<D, T, 2, true>), dim3((unsigned)blocks),
                           dim3(kRowWaves * 2 * 64), 0, stream, params);
      else
        return hipErrorInvalidValue;
    }
  } else if constexpr (D > 128) {
    if (params.groups != 1) return hipErrorInvalidValue;
    hipLaunchKernelGGL((paged_prefill_kernel<D, T, 1, false>), dim3((unsigned)blocks), dim3(kRowWaves * 64), 0, stream, params);
  } else if (params.groups == 1) {
    hipLaunchKernelGGL((paged_prefill_kernel<D, T, 1, false>), dim3((unsigned)blocks), dim3(kRowWaves * 64), 0, stream, params);
  } else if (params.groups == 2) {
    hipLaunchKernelGGL((paged_prefill_kernel<D, T, 2, false>), dim3((unsigned)blocks), dim3(kRowWaves * 2 * 64), 0, stream,
                       params);
  } else {
    return hipErrorInvalidValue;
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || params.kv_splits == 1) return err;
  const int64_t split_pairs = (int64_t)(params.seq_count ? params.seq_count : params.num_seqs) * params.num_kv_heads;
  hipLaunchKernelGGL((prefill_merge_kernel<D, T, TT>),
                     dim3((unsigned)(split_pairs * params.row_tiles * (kBlockRows / (kMergeWaves * merge_rows<D>())))),
                     dim3(256), 0, stream, params);
  return hipGetLastError();
}

} // namespace

hipError_t launch_paged_prefill(const PrefillParams& params, int head_dim, bool f32, hipStream_t stream) {
  if (!prefill_head_dim_supported(head_dim)) return hipErrorInvalidValue;
  if (f32) {
    if (head_dim == 128) return launch_typed<128, float>(params, stream);
    if (head_dim == 64) return launch_typed<64, float>(params, stream);
    if (head_dim == 32) return launch_typed<32, float>(params, stream);
    if (head_dim == 96) return launch_typed<96, float>(params, stream);
    if (head_dim == 160) return launch_typed<160, float>(params, stream);
    if (head_dim == 192) return launch_typed<192, float>(params, stream);
    if (head_dim == 224) return launch_typed<224, float>(params, stream);
    if (head_dim == 256) return launch_typed<256, float>(params, stream);
  } else {
    if (head_dim == 128) return launch_typed<128, half_t>(params, stream);
    if (head_dim == 64) return launch_typed<64, half_t>(params, stream);
    if (head_dim == 32) return launch_typed<32, half_t>(params, stream);
    if (head_dim == 96) return launch_typed<96, half_t>(params, stream);
    if (head_dim == 160) return launch_typed<160, half_t>(params, stream);
    if (head_dim == 192) return launch_typed<192, half_t>(params, stream);
    if (head_dim == 224) return launch_typed<224, half_t>(params, stream);
    if (head_dim == 256) return launch_typed<256, half_t>(params, stream);
  }
  return hipErrorInvalidValue;
}

} // namespace mvr
