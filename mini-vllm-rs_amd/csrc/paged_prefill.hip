// Chunked-prefill page-wise attention for gfx950 (F16, MFMA 32x32x16).
//
// Same contract as paged_attention.hip (common.rs:739-817 semantics: grouped
// rows rho = r*q_len + i, key j visible to query i iff j <= seq_len - q_len + i)
// for requests with many query rows per KV head, where attention is a dense
// contraction (about 950 flop per byte of K/V at q_len 256) and the MFMA
// pipes, not HBM, set the roofline.
//
// Block = 4 wavefronts = 128 consecutive grouped rows of one (sequence, KV
// head); the block walks the visible keys in 32-token tiles that all four
// wavefronts share through LDS (a ring of kStages stages, 16 KiB per stage at
// D=128, filled by direct-to-LDS loads):
//   * K tile: 16-byte chunks, XOR swizzle (chunk ^ row%16), read back with
//     ds_read_b128 in the v_mfma_f32_32x32x16_f16 A-operand layout
//     (lane l: token l%32, dims 8*(l/32)+16s);  S^T = K Q^T in D/16 MFMAs;
//   * S^T lands with lane l owning row l%32 and 16 tokens; the online softmax
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

constexpr int kTileTokens = 32;
constexpr int kRowsPerWave = 32;
constexpr int kWaves = 4;
constexpr int kBlockRows = kRowsPerWave * kWaves;
constexpr int kXcds = 8;
#ifndef MVR_PREFILL_STAGES
#define MVR_PREFILL_STAGES 4
#endif
constexpr int kStages = MVR_PREFILL_STAGES; // LDS stages (4 or 8): the unrolled loop names each statically
constexpr float kRescaleThreshold = 8.0f; // log2 units: p <= 2^8 between rescales

struct SeqRows {
  int seq_len, q_start, q_len, key_end; // keys [0, key_end) belong to this call
};

// Tile barrier: waits until at most kNewer of this wavefront's direct-to-LDS
// tile loads are in flight and its LDS reads have returned, then meets the
// other wavefronts.  (__syncthreads() would wait for every load, vmcnt(0),
// and drain the prefetch.)  The wait is the compiler's own s_waitcnt, so its
// bookkeeping of the direct-to-LDS loads stays exact; the empty asm
// statements keep memory accesses from moving across the barrier without
// any further wait.
// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane
// (global_load_lds_dwordx4).  A plain __device__ function: lambdas in kernels
// are also compiled for the host, where this gfx950 builtin does not exist.
__device__ __forceinline__ void load_to_lds16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void*)lds, 16, 0, 0);
}

template <int kNewer>
__device__ __forceinline__ void tile_barrier() {
  __builtin_amdgcn_s_waitcnt((kNewer & 0xF) | ((kNewer >> 4) << 14) | (0x7 << 4)); // vmcnt(n) expcnt(7) lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ SeqRows load_rows(const PrefillParams& p, int b) {
  SeqRows s;
  s.seq_len = p.seq_lens ? p.seq_lens[b] : p.single_seq_len;
  if (p.cu_q_lens) {
    s.q_start = p.cu_q_lens[b];
    s.q_len = p.cu_q_lens[b + 1] - s.q_start;
  } else {
    s.q_start = 0;
    s.q_len = p.single_q_len;
  }
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

// Keys the block's rows can see: up to the largest causal limit among them.
__device__ __forceinline__ int block_key_tiles(const SeqRows& s, int group_size, int rt) {
  const int rows = group_size * s.q_len;
  const int rho0 = rt * kBlockRows;
  if (rho0 >= rows || s.q_len <= 0) return 0;
  const int rho1 = min(rho0 + kBlockRows, rows) - 1;
  const int max_i = (rho1 / s.q_len != rho0 / s.q_len) ? s.q_len - 1 : rho1 % s.q_len;
  const int last_key = row_limit(s, max_i); // -1: no key (a prefix pass over an empty prefix)
  return last_key < 0 ? 0 : last_key / kTileTokens + 1;
}

template <int D>
struct Tile {
  static constexpr int kChunksPerRow = D / 8;                          // 16-byte chunks per token row
  static constexpr int kChunks = kTileTokens * kChunksPerRow;          // per K (or V) tile
  static constexpr int kChunksPerThread = kChunks / (kWaves * 64);     // 2 at D=128, 1 at D=64
  static constexpr int kElems = kTileTokens * D;
  // V: 32-byte pieces per row, XOR-swizzled with the row.  A transposed read
  // is served per half-wavefront: 4 rows x 2 adjacent pieces, which must land
  // in 8 distinct 32-byte bank groups; 2*(row&3) (D=128) spreads the 4 piece
  // pairs apart, measured conflict-free on gfx950 (row&7 cost 2 extra
  // cycles per read).  At D=64 two rows share a 256-byte bank line and
  // row&3 is already conflict-free.
  __device__ static __forceinline__ int vswz(int t) { return D == 128 ? 2 * (t & 3) : (t & 3); }
  __device__ static __forceinline__ int kswz(int t) { return t & (kChunksPerRow - 1); }
};

template <int D>
__global__ __launch_bounds__(kWaves * 64, D == 128 ? 1 : 2) void paged_prefill_kernel(PrefillParams p) {
  typedef Tile<D> TL;
  // One LDS object per stage and operand: the compiler tracks the
  // direct-to-LDS loads per object, so a read of one stage never waits for
  // the loads still landing in another.
  __shared__ __attribute__((aligned(16))) half_t k_lds0[TL::kElems], k_lds1[TL::kElems], k_lds2[TL::kElems],
      k_lds3[TL::kElems], k_lds4[TL::kElems], k_lds5[TL::kElems], k_lds6[TL::kElems], k_lds7[TL::kElems];
  __shared__ __attribute__((aligned(16))) half_t v_lds0[TL::kElems], v_lds1[TL::kElems], v_lds2[TL::kElems],
      v_lds3[TL::kElems], v_lds4[TL::kElems], v_lds5[TL::kElems], v_lds6[TL::kElems], v_lds7[TL::kElems];

  const int tid = threadIdx.x;
  const int l = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int hh = l >> 5; // lane half: 0 or 1

  // XCD-aware decode of the block index: block x runs on XCD x % 8; all
  // blocks of one (sequence, kv head) pair sit on the same XCD.
  // With fewer pairs than XCDs, plain linear order keeps every XCD busy.
  const int x = blockIdx.x;
  const int per_pair = p.row_tiles * p.kv_splits;
  const int pairs = p.num_seqs * p.num_kv_heads;
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
  const int b = pair / p.num_kv_heads;
  const int split = local % p.kv_splits;
  const int rt = local / p.kv_splits;

  const SeqRows s = load_rows(p, b);
  const int rows = p.group_size * s.q_len;
  const int n_tiles = block_key_tiles(s, p.group_size, rt);
  if (n_tiles == 0) return; // whole block: uniform exit before any barrier
  const int tiles_per_split = (n_tiles + p.kv_splits - 1) / p.kv_splits;
  const int j0 = split * tiles_per_split;
  const int j1 = min(j0 + tiles_per_split, n_tiles);
  const int64_t slot = (int64_t)((b * p.num_kv_heads + h) * p.row_tiles + rt) * p.kv_splits + split;

  // This lane's query row.
  const int rho = rt * kBlockRows + wave * kRowsPerWave + (l & 31);
  const bool valid = rho < rows;
  const int r = valid ? rho / s.q_len : 0;
  const int i = valid ? rho % s.q_len : 0;
  const int limit = valid ? row_limit(s, i) : -1;
  // Largest causal limit among the wave's rows (rows of a wave are contiguous).
  int wave_limit = limit;
  for (int off = 1; off < 64; off <<= 1) wave_limit = max(wave_limit, __shfl_xor(wave_limit, off));
  int wave_min_limit = valid ? limit : INT32_MAX;
  for (int off = 1; off < 64; off <<= 1) wave_min_limit = min(wave_min_limit, __shfl_xor(wave_min_limit, off));

  // Q^T as the B operand: lane l holds Q[rho][16s + 8*hh .. +8].
  half8 q[D / 16];
  {
    const half_t* qrow = static_cast<const half_t*>(p.q) + (int64_t)(h * p.group_size + r) * p.q_stride_head +
                         (int64_t)(s.q_start + i) * p.q_stride_token;
#pragma unroll
    for (int st = 0; st < D / 16; st++) q[st] = valid ? *reinterpret_cast<const half8*>(qrow + 16 * st + 8 * hh) : half8{};
  }

  float16v o[D / 32];
#pragma unroll
  for (int n = 0; n < D / 32; n++)
#pragma unroll
    for (int e = 0; e < 16; e++) o[n][e] = 0.f;
  float m = -INFINITY, lsum = 0.f;

  const half_t* kpool = static_cast<const half_t*>(p.key_pool);
  const half_t* vpool = static_cast<const half_t*>(p.value_pool);
  // Block-table reads use the constant address space with a wave-uniform
  // index, so they are scalar loads and never wait on the K/V loads in flight.
  const const_i32* bt = (const const_i32*)(p.block_tables) + (int64_t)b * p.block_table_stride;

  // Page arithmetic by shifts: the host routes only power-of-two page sizes
  // (multiples of 16) to this kernel.
  const int pshift = p.page_shift;
  auto page_div = [&](int tok) { return tok >> pshift; };
  auto page_mod = [&](int tok) { return tok & (p.page_size - 1); };

  // Tiles move straight from HBM/L2 into LDS (global_load_lds_dwordx4: lane
  // i of a wavefront writes 16 bytes at the wavefront's LDS base + 16 i), so
  // they take no registers and no LDS store instructions.  Wavefront w, step
  // u fills LDS chunks (u*4 + w)*64 .. +63 of a tile; LDS chunk P holds token
  // row t = P / (D/8), physical chunk P % (D/8), and the lane fetches the
  // logical 16-byte chunk that the K or V swizzle puts there.  The tokens of
  // one (w, u) are 4 (D=128) or 8 (D=64) consecutive tokens of a 16-token
  // group, hence of one page: one scalar block-table load per (w, u).
  int ld_t[TL::kChunksPerThread], ld_t0[TL::kChunksPerThread], ld_k[TL::kChunksPerThread],
      ld_v[TL::kChunksPerThread];
#pragma unroll
  for (int u = 0; u < TL::kChunksPerThread; u++) {
    const int P = (u * kWaves + wave) * 64 + l;
    const int t = P / TL::kChunksPerRow, cs = P % TL::kChunksPerRow;
    ld_t[u] = t;
    ld_t0[u] = (u * kWaves + wave) * 64 / TL::kChunksPerRow;
    ld_k[u] = 8 * (cs ^ TL::kswz(t));
    ld_v[u] = 8 * (2 * ((cs >> 1) ^ TL::vswz(t)) + (cs & 1));
  }
  // Branch-free: tokens past the call's last key re-read that key,
  // so every tile issues the same loads.  Those duplicate keys lie past every
  // row's causal limit (the last tile is a diagonal tile for every wavefront
  // that sees it), so their scores are masked to -inf, p = 0, and
  // p * (finite duplicate V) = 0.
  // Block-table entries of a tile's (w, u) groups, read one iteration before
  // the tile's loads are issued: a scalar load makes its user wait for
  // lgkmcnt(0), which would also drain every LDS read in flight, so the
  // entries are fetched just before a barrier, where lgkmcnt is drained anyway.
  struct Pages {
    int64_t pg[TL::kChunksPerThread];
  };
  auto fetch_pages = [&](int j) {
    Pages r;
#pragma unroll
    for (int u = 0; u < TL::kChunksPerThread; u++)
      r.pg[u] = bt[page_div(min(j * kTileTokens + ld_t0[u], s.key_end - 1))]; // wave-uniform: scalar load
    return r;
  };
  auto issue_tile = [&](int j, const Pages& pages, half_t* kb, half_t* vb) {
#pragma unroll
    for (int u = 0; u < TL::kChunksPerThread; u++) {
      const int tg = min(j * kTileTokens + ld_t[u], s.key_end - 1);
      const int64_t row = ((pages.pg[u] * p.num_kv_heads + h) * p.page_size + page_mod(tg)) * D;
      const int dst = (u * kWaves + wave) * 64 * 8;
      load_to_lds16(kpool + row + ld_k[u], kb + dst);
      load_to_lds16(vpool + row + ld_v[u], vb + dst);
    }
  };
  constexpr int kLoadsPerTile = 2 * TL::kChunksPerThread; // per lane
  half_t* const k_st[8] = {k_lds0, k_lds1, k_lds2, k_lds3, k_lds4, k_lds5, k_lds6, k_lds7};
  half_t* const v_st[8] = {v_lds0, v_lds1, v_lds2, v_lds3, v_lds4, v_lds5, v_lds6, v_lds7};

  // Per-lane LDS read offsets, loop-invariant.  K: lane reads token l%32,
  // chunk 2s+hh.  V^T: step u reads rows 16u+4hh+rsub (and +8), 16 columns
  // at 32n+16*(g16&1)+csub, through the transposing read.
  int rk[D / 16];
  {
    const int t = l & 31;
#pragma unroll
    for (int st = 0; st < D / 16; st++) rk[st] = t * D + 8 * ((2 * st + hh) ^ TL::kswz(t));
  }
  int rva[D / 32][2], rvb[D / 32][2];
  {
    const int g16 = l >> 4, qd = l & 15;
    const int rsub = qd >> 2, csub = 4 * (qd & 3);
#pragma unroll
    for (int n = 0; n < D / 32; n++)
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int row_a = 16 * u + 4 * hh + rsub, row_b = row_a + 8;
        const int col = 32 * n + 16 * (g16 & 1) + csub;
        rva[n][u] = row_a * D + ((col >> 4) ^ TL::vswz(row_a)) * 16 + (col & 15);
        rvb[n][u] = row_b * D + ((col >> 4) ^ TL::vswz(row_b)) * 16 + (col & 15);
      }
  }
  const float sl2 = p.scale_log2;

  // Wave-uniform tile predicates: a tile is visible when some row of this
  // wavefront sees its first key, and diagonal when some row does not see
  // its last key (then scores are masked).
  auto visible = [&](int j) { return j < j1 && j * kTileTokens <= wave_limit; };
  auto diagonal = [&](int j) { return j * kTileTokens + kTileTokens - 1 > wave_min_limit; };

  // S^T of the tile in stage buf: D/16 MFMAs, K read straight into the A operand.
  auto qk = [&](const half_t* kb) {
    float16v acc;
#pragma unroll
    for (int e = 0; e < 16; e++) acc[e] = 0.f;
#pragma unroll
    for (int st = 0; st < D / 16; st++)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8*>(kb + rk[st]), q[st], acc, 0, 0, 0);
    return acc;
  };
  // Lane holds tokens tok0 + 8*(e/4) + 4*hh + e%4 of row rho.
  auto mask = [&](int j, float16v& sv) {
    const int rel = limit - j * kTileTokens - 4 * hh;
#pragma unroll
    for (int e = 0; e < 16; e++) sv[e] = 8 * (e >> 2) + (e & 3) <= rel ? sv[e] : -INFINITY;
  };
  // Scaled row max (log2 units; scale > 0 keeps the order), both lane halves.
  auto row_max = [&](const float16v& sv) {
    float a = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    float b = fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7]));
    float c = fmaxf(fmaxf(sv[8], sv[9]), fmaxf(sv[10], sv[11]));
    float d = fmaxf(fmaxf(sv[12], sv[13]), fmaxf(sv[14], sv[15]));
    const float mx = fmaxf(fmaxf(a, b), fmaxf(c, d)) * sl2;
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
  auto exps = [&](const float16v& sv, half8 (&pb)[2]) {
    const float neg_m = m == -INFINITY ? 0.f : -m;
    float psum = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const float pe = __builtin_amdgcn_exp2f(fmaf(sv[e], sl2, neg_m));
      psum += pe;
      pb[e >> 3][e & 7] = (half_t)pe;
    }
    lsum += psum;
  };
  // O^T += V^T P^T over two 16-token steps u; step u uses tokens
  // 16u + 4*hh + {0..3} and 16u + 8 + 4*hh + {0..3} (the ones this lane holds).
  auto pv = [&](const half_t* vb, const half8 (&pb)[2]) {
#pragma unroll
    for (int n = 0; n < D / 32; n++) {
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const short4v ra = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vb + rva[n][u]));
        const short4v rb = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(vb + rvb[n][u]));
        const half8 vt = __builtin_bit_cast(half8, __builtin_shufflevector(ra, rb, 0, 1, 2, 3, 4, 5, 6, 7));
        o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vt, pb[u], o[n], 0, 0, 0);
      }
    }
  };

  // Software pipeline over 32-token tiles in kStages LDS stages; the stage of
  // tile t is (t - j0) % kStages.  Iteration j issues the loads of tile
  // j + kStages - 1 into the stage that held tile j-1 (released by the
  // previous barrier), so every tile has kStages - 2 iterations to arrive.
  // Then, with tile j's scores sc already masked and folded into the running
  // max:
  //   block A: S(j+1) = K(j+1) Q^T on the MFMA pipe while the VALU computes
  //            P(j) = exp2(sc - m) (independent instructions, one basic block);
  //   block B: O += V(j)^T P(j) on the MFMA pipe while the VALU masks and
  //            reduces S(j+1);
  // moves the running max for tile j+1, and the wavefronts meet once tile
  // j+2 has landed.  Loads past the last tile re-read it (clamped) into
  // stages nobody reads again.  Measured on the Qwen2-7B prefill chunk: 4
  // stages 70 us, 8 stages 84 us (more loads in flight slowed the block).
  constexpr int kAhead = kStages - 1;                        // tiles issued ahead of the one consumed
  constexpr int kInFlight = (kStages - 3) * kLoadsPerTile;   // loads a barrier leaves in flight
  const int j_last = max(j1 - 1, j0);
#pragma unroll
  for (int a = 0; a < kAhead; a++) {
    const int t = min(j0 + a, j_last);
    issue_tile(t, fetch_pages(t), k_st[a], v_st[a]);
  }
  Pages next_pages = fetch_pages(min(j0 + kAhead, j_last));
  tile_barrier<kInFlight + kLoadsPerTile>(); // tiles j0 and j0+1 landed

  float16v sc;
#pragma unroll
  for (int e = 0; e < 16; e++) sc[e] = 0.f;
  if (visible(j0)) {
    sc = qk(k_st[0]);
    if (diagonal(j0)) mask(j0, sc);
    advance_max(row_max(sc));
  }

  // Tiles every row of the block sees in full need neither visibility tests
  // nor masks; while tiles j and j+1 are both such, an iteration is one
  // branch-free stretch.
  auto iterate_clear = [&](int j, auto st_c) {
    constexpr int st = decltype(st_c)::value;
    issue_tile(min(j + kAhead, j_last), next_pages, k_st[(st + kAhead) & (kStages - 1)],
               v_st[(st + kAhead) & (kStages - 1)]);
    half8 pb[2];
    const float16v sn = qk(k_st[(st + 1) & (kStages - 1)]);
    exps(sc, pb);
    pv(v_st[st], pb);
    advance_max(row_max(sn));
    sc = sn;
    next_pages = fetch_pages(min(j + kStages, j_last));
    tile_barrier<kInFlight>();
  };
  auto iterate = [&](int j, auto st_c) {
    constexpr int st = decltype(st_c)::value;
    issue_tile(min(j + kAhead, j_last), next_pages, k_st[(st + kAhead) & (kStages - 1)],
               v_st[(st + kAhead) & (kStages - 1)]);
    if (visible(j)) {
      half8 pb[2];
      if (visible(j + 1)) {
        float16v sn = qk(k_st[(st + 1) & (kStages - 1)]);
        exps(sc, pb);
        if (diagonal(j + 1)) mask(j + 1, sn);
        pv(v_st[st], pb);
        advance_max(row_max(sn));
        sc = sn;
      } else {
        exps(sc, pb);
        pv(v_st[st], pb);
      }
    }
    next_pages = fetch_pages(min(j + kStages, j_last));
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
  // Clear iterations need j + 1 clear as well; their count is a multiple of
  // kStages so that the general loop starts on stage 0.
  const int j_mid = j0 + max(0, (clear_tiles - 1 - j0) / kStages * kStages);

  // Unrolled by kStages so that every stage is named statically: LDS
  // addresses become immediate offsets and each stage is its own object.
#define MVR_STAGE(K) std::integral_constant<int, K>()
  for (int j = j0; j < j_mid; j += kStages) {
    iterate_clear(j, MVR_STAGE(0));
    iterate_clear(j + 1, MVR_STAGE(1));
    iterate_clear(j + 2, MVR_STAGE(2));
    iterate_clear(j + 3, MVR_STAGE(3));
    if constexpr (kStages == 8) {
      iterate_clear(j + 4, MVR_STAGE(4));
      iterate_clear(j + 5, MVR_STAGE(5));
      iterate_clear(j + 6, MVR_STAGE(6));
      iterate_clear(j + 7, MVR_STAGE(7));
    }
  }
  for (int j = j_mid; j < j1; j += kStages) {
    iterate(j, MVR_STAGE(0));
    if (j + 1 >= j1) break;
    iterate(j + 1, MVR_STAGE(1));
    if (j + 2 >= j1) break;
    iterate(j + 2, MVR_STAGE(2));
    if (j + 3 >= j1) break;
    iterate(j + 3, MVR_STAGE(3));
    if constexpr (kStages == 8) {
      if (j + 4 >= j1) break;
      iterate(j + 4, MVR_STAGE(4));
      if (j + 5 >= j1) break;
      iterate(j + 5, MVR_STAGE(5));
      if (j + 6 >= j1) break;
      iterate(j + 6, MVR_STAGE(6));
      if (j + 7 >= j1) break;
      iterate(j + 7, MVR_STAGE(7));
    }
  }
#undef MVR_STAGE
  // Every issued load has landed before the block exits (the last barrier
  // left up to one tile of clamped re-reads in flight).
  __builtin_amdgcn_s_waitcnt(0x0070); // vmcnt(0) expcnt(7) lgkmcnt(0)

  const float ltot = lsum + __shfl_xor(lsum, 32);
  // Lane holds O^T[d][rho] for d = 32n + 8*(e/4) + 4*hh + e%4.
  if (p.kv_splits == 1) {
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
    } else if (valid) {
      const float inv = 1.f / ltot;
      half_t* dst = static_cast<half_t*>(p.out) + (int64_t)(h * p.group_size + r) * p.out_stride_head +
                    (int64_t)(s.q_start + i) * p.out_stride_token;
#pragma unroll
      for (int n = 0; n < D / 32; n++)
#pragma unroll
        for (int a = 0; a < 4; a++) {
          half4 v4 = {(half_t)(o[n][4 * a] * inv), (half_t)(o[n][4 * a + 1] * inv), (half_t)(o[n][4 * a + 2] * inv),
                      (half_t)(o[n][4 * a + 3] * inv)};
          *reinterpret_cast<half4*>(dst + 32 * n + 8 * a + 4 * hh) = v4;
        }
    }
  } else if (valid) {
    const int64_t prow = slot * kBlockRows + wave * kRowsPerWave + (l & 31);
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

// Merges the kv_splits partial results of every block tile:
//   out = sum_j 2^(m_j - M) o_j / sum_j 2^(m_j - M) l_j.
// One wavefront per output row (a 256-thread block covers 4 rows of a tile):
// lane j holds split j's weight, broadcast by readlane while the partial rows
// stream as one coalesced 4*D-byte row per load.  Empty splits (no visible
// key) hold m = -inf, l = 0 and weigh nothing.
template <int D>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillParams p) {
  constexpr int kPer = D / 64;
  constexpr int kBlocksPerTile = kBlockRows / kWaves;
  const int tile = blockIdx.x / kBlocksPerTile; // (b, h, rt)
  const int lr = (blockIdx.x % kBlocksPerTile) * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  const int rt = tile % p.row_tiles;
  const int h = (tile / p.row_tiles) % p.num_kv_heads;
  const int b = tile / (p.row_tiles * p.num_kv_heads);
  const SeqRows s = load_rows(p, b);
  const int rho = rt * kBlockRows + lr;
  if (rho >= p.group_size * s.q_len) return;
  const int n_tiles = block_key_tiles(s, p.group_size, rt);
  if (n_tiles == 0) return;
  const int tiles_per_split = (n_tiles + p.kv_splits - 1) / p.kv_splits;
  const int n_parts = (n_tiles + tiles_per_split - 1) / tiles_per_split; // splits that ran (<= 8 < 64 lanes)
  const int64_t prow0 = (int64_t)tile * p.kv_splits * kBlockRows + lr;  // split j: prow0 + j * kBlockRows
  const float mj = l < n_parts ? p.partial_ml[(prow0 + (int64_t)l * kBlockRows) * 2] : -INFINITY;
  float mmax = mj;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mmax = fmaxf(mmax, __shfl_xor(mmax, off));
  const float m_use = mmax == -INFINITY ? 0.f : mmax;
  const float w = mj == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mj - m_use);
  float den = l < n_parts ? w * p.partial_ml[(prow0 + (int64_t)l * kBlockRows) * 2 + 1] : 0.f;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) den += __shfl_xor(den, off);
  float acc[kPer];
#pragma unroll
  for (int e = 0; e < kPer; e++) acc[e] = 0.f;
  for (int j = 0; j < n_parts; j++) {
    const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), j));
    const float* src = p.partial_o + (prow0 + (int64_t)j * kBlockRows) * D + l * kPer;
#pragma unroll
    for (int e = 0; e < kPer; e++) acc[e] = fmaf(wj, src[e], acc[e]);
  }
  const int r = rho / s.q_len, i = rho % s.q_len;
  const float inv = 1.f / den;
  if (p.state_o) {
    const int64_t srow = (int64_t)(h * p.group_size + r) * p.state_tokens + s.q_start + i;
#pragma unroll
    for (int e = 0; e < kPer; e++) p.state_o[srow * D + l * kPer + e] = acc[e] * inv;
    if (l == 0) p.state_lse[srow] = m_use + __log2f(den);
    return;
  }
  half_t* dst = static_cast<half_t*>(p.out) + (int64_t)(h * p.group_size + r) * p.out_stride_head +
                (int64_t)(s.q_start + i) * p.out_stride_token + l * kPer;
#pragma unroll
  for (int e = 0; e < kPer; e++) dst[e] = (half_t)(acc[e] * inv);
}

template <int D>
hipError_t launch_typed(const PrefillParams& params, hipStream_t stream) {
  const int pairs = params.num_seqs * params.num_kv_heads;
  const int per_pair = params.row_tiles * params.kv_splits;
  const int64_t blocks =
      pairs >= kXcds ? (int64_t)kXcds * ((pairs + kXcds - 1) / kXcds) * per_pair : (int64_t)pairs * per_pair;
  hipLaunchKernelGGL(paged_prefill_kernel<D>, dim3((unsigned)blocks), dim3(kWaves * 64), 0, stream, params);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || params.kv_splits == 1) return err;
  hipLaunchKernelGGL(prefill_merge_kernel<D>, dim3(pairs * params.row_tiles * (kBlockRows / kWaves)), dim3(256), 0,
                     stream, params);
  return hipGetLastError();
}

} // namespace

hipError_t launch_paged_prefill(const PrefillParams& params, int head_dim, hipStream_t stream) {
  if (head_dim == 128) return launch_typed<128>(params, stream);
  if (head_dim == 64) return launch_typed<64>(params, stream);
  return hipErrorInvalidValue;
}

} // namespace mvr
