// Paged-A KV cache <-> token-major linear transfers for MI355X (gfx950):
// 16- and 32-bit copies, and the dispatch of every paged-A transfer.
//
// Cache layout (the reference API layout, musa_aiter/ops/kv_transfer.py:3-14):
//   [NL, NB, NH, HD, BS]  -- block_size innermost, so one token's head row is
//   strided by BS elements.  Linear layout: [.., T, NH, HD] token-major rows.
//
// Design.  A "run" is a maximal set of consecutive tokens whose slots are
// consecutive inside one block (tokens of one sequence filling one block).
// For one run, the block's rows [r0, r0 + kRows) are a contiguous 4 KiB
// region of the cache and a [BS tokens x kRows] slab of the linear rows: a
// small 2-D transpose.  One 256-thread workgroup owns the runs that start in
// its 16-token tile, for one such row chunk of one (layer, K|V) plane:
//   * every thread moves exactly one 16-byte cache piece (whole lines per
//     wave instruction) and one 16-byte linear piece (RPL rows of one token,
//     256-1024 contiguous bytes per token per wave instruction);
//   * the two orientations meet in a padded LDS tile: cache pieces are
//     written/read as rows, linear pieces as RPL column elements.
// Each wave keeps at most a few hundred bytes per lane in flight and lives for
// one chunk, the access shape that reaches the highest HBM copy rate on
// MI355X.  Partial runs store only their own block columns (element stores at
// the edges), so neighbouring slots are never touched.  Skipped tokens
// (slot < 0) are zero filled by the workgroup that owns them.  FP8 caches go
// to the per-wave kernels of kv_paged_waves.hip; any shape or alignment the
// tiled kernels do not cover goes to the element-wise kernel below.
#include "kv_hip_common.h"
#include "kv_launch.h"
#include "kv_paged_args.h"

#include <type_traits>

namespace kvhip {

// ----- the cooperative tile kernel (16- and 32-bit copies) ----------------------------

constexpr int kCoopThreads = 256;

template <int ELT, int BS, int NT = kCoopThreads>
struct CoopShape {
  static constexpr int CG = 16 / ELT;                 // block columns per cache piece
  static constexpr int NCG = BS / CG;                 // cache pieces per cache row
  static constexpr int ROWB = BS * ELT;               // bytes per cache row of a block
  static constexpr int kRows = NT * 16 / ROWB;        // cache rows per chunk (NT x 16 bytes)
  static constexpr int RPL = 16 / ELT;                // rows per linear piece
  static constexpr int G = kRows / RPL;               // linear pieces per token per chunk
  static constexpr int PITCH = ROWB + 4;              // LDS bytes per cache row (one pad dword)
  static_assert(BS % CG == 0, "block row must be a whole number of 16-byte pieces");
  static_assert(BS * G == NT, "linear pieces must cover the chunk");
  static_assert(G % 8 == 0, "row groups come in eights");

  // Linear piece p of a chunk -> (block column, row group).  Eight
  // consecutive pieces are eight row groups of one token (128 contiguous
  // bytes of its row); a wave covers eight tokens.  In the LDS tile the
  // eight row groups of a wave start 8 rows apart, which with the padded
  // pitch spreads a column read over distinct banks.
  __device__ static __forceinline__ int col(int p) { return (p >> 3) % BS; }
  __device__ static __forceinline__ int grp(int p) { return (p & 7) + 8 * (p / (8 * BS)); }
};

// Linear piece (RPL rows of block column c) assembled from the LDS tile.
template <int ELT, int PITCH>
__device__ __forceinline__ u32x4 lds_column_piece(const uint8_t* tile, int row0, int c) {
  const uint8_t* p = tile + row0 * PITCH + c * ELT;
  u32x4 o;
  if constexpr (ELT == 2) {
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = pack16(load_elem<2>(p + (2 * k) * PITCH), load_elem<2>(p + (2 * k + 1) * PITCH));
  } else {
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = load_elem<4>(p + k * PITCH);
  }
  return o;
}

// Writes the RPL elements of one linear piece into column c of the LDS tile.
template <int ELT, int PITCH>
__device__ __forceinline__ void lds_put_column(uint8_t* tile, int row0, int c, const u32x4& in) {
  constexpr int RPL = 16 / ELT;
  uint8_t* p = tile + row0 * PITCH + c * ELT;
#pragma unroll
  for (int i = 0; i < RPL; ++i) store_elem<ELT>(p + i * PITCH, piece_elem<ELT>(in, i));
}

// Workgroup barrier for the LDS tile only: waits for this wave's LDS
// accesses, not for its outstanding global loads (the next chunk's prefetch
// stays in flight across the barrier).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Chunks of one run handled by one workgroup (grid z covers the rest): the
// gather does best with more, shorter-lived workgroups, the scatter (whose
// setup includes the claim check) with longer ones (measured).
template <bool SCATTER>
constexpr int kChunksPerGroup = SCATTER ? 4 : 2;

// One run of a large scatter (block columns [c0, c1) of the block at `cbuf`,
// linear rows of its first token at `lbuf`, both at the workgroup's first
// row), chunk by chunk with the next chunk's load in flight (2 % faster than
// issuing every load first when the grid is many rounds of workgroups,
// measured; their time is the cache writes).  CSTP: cache policy of the
// stores of runs that fill the whole block (every line of the chunk written
// at once); partial runs store non-temporally.  Ends with the LDS tile free.
template <int ELT, int BS, int NT, int CSTP = kBufNT>
__device__ __forceinline__ void scatter_run_chunks(uint8_t* tile, buf_t cbuf, buf_t lbuf, int c0, int c1,
                                                   int nchunks, int rows_left, uint32_t stride32) {
  using S = CoopShape<ELT, BS, NT>;
  constexpr int CG = S::CG, NCG = S::NCG, ROWB = S::ROWB, kRows = S::kRows;
  constexpr int RPL = S::RPL, PITCH = S::PITCH;
  const int tid = static_cast<int>(threadIdx.x);
  const int pr = tid / NCG;
  const int pg = tid % NCG;
  const int lc = S::col(tid);
  const int lq = S::grp(tid);
  constexpr uint32_t kCacheStep = kRows * ROWB;
  constexpr uint32_t kLinStep = kRows * ELT;
  const uint32_t cpiece = static_cast<uint32_t>(tid) * 16u;
  const bool lmine = lc >= c0 && lc < c1;
  const uint32_t lbase = static_cast<uint32_t>(lc - c0) * stride32 + static_cast<uint32_t>(lq) * 16u;
  auto coff = [&](int k) -> uint32_t { return k * kRows + pr < rows_left ? cpiece + k * kCacheStep : kOffOob; };
  auto lrow_in = [&](int k) { return k * kRows + lq * RPL < rows_left; };
  auto loff = [&](int k) -> uint32_t { return (lmine && lrow_in(k)) ? lbase + k * kLinStep : kOffOob; };
  u32x4 nxt = buf_ld16(lbuf, loff(0));
  const bool full_run = (c0 == 0) && (c1 == BS);
  for (int k = 0; k < nchunks; ++k) {
    const u32x4 in = nxt;
    nxt = buf_ld16(lbuf, (k + 1 < nchunks) ? loff(k + 1) : kOffOob);
    if (lmine && lrow_in(k)) lds_put_column<ELT, PITCH>(tile, lq * RPL, lc, in);
    lds_barrier();
    const uint32_t* const d = reinterpret_cast<const uint32_t*>(tile + pr * PITCH + pg * 16);
    const u32x4 w = {d[0], d[1], d[2], d[3]};
    const uint32_t off = coff(k);
    const int lo = pg * CG;
    if (full_run) {
      buf_st16_p<CSTP>(cbuf, off, w);
    } else {
      const bool whole = lo >= c0 && lo + CG <= c1;
      buf_st16(cbuf, whole ? off : kOffOob, w);
#pragma unroll
      for (int cc = 0; cc < CG; ++cc) {
        const bool mine = !whole && off != kOffOob && lo + cc >= c0 && lo + cc < c1;
        buf_st_elem<ELT>(cbuf, mine ? off + cc * ELT : kOffOob, piece_elem<ELT>(w, cc));
      }
    }
    lds_barrier();
  }
}

// Tiles of short runs (one or a few tokens per block, as a decode step's one
// new token per sequence) skip the LDS transpose, which costs one load round
// trip and 2 x C workgroup barriers per run.  Wave w takes tokens
// w, w + W, ... of the tile (W waves) and, per 64-row block of the group [rb,
// re), moves row (block * 64 + lane) of the token: one instruction covers 64
// consecutive rows, one 128-byte line of the linear row (16-bit elements) and
// 16 lines of the block column.  The token is wave-uniform, so its linear row
// and block column are scalar buffer descriptors.  Lane i + 1 of `s` holds the
// slot of token t0 + i; bit i + 1 of `vw` (bits 1..kTileTokens) says that the
// token moves.  Every load of a batch (up to 32 rows per lane) is issued
// before its stores.
template <int ELT, int BS, int NT, bool SCATTER>
__device__ __forceinline__ void token_rows(const TileArgs& a, uint8_t* cache, uint8_t* lin, int64_t s, uint64_t vw,
                                           int64_t t0, int64_t rb, int64_t re) {
  constexpr int ROWB = BS * ELT;
  constexpr int kGroupRows = CoopShape<ELT, BS, NT>::kRows * kChunksPerGroup<SCATTER>;
  static_assert(kGroupRows % kWave == 0, "row blocks of one wave");
  constexpr int NRB = kGroupRows / kWave;   // 64-row blocks per token
  constexpr int kWaves = NT / kWave;
  constexpr int TPW = kTileTokens / kWaves;  // tokens per wave
  constexpr int TB = TPW * NRB <= 32 ? TPW : 32 / NRB;  // tokens per batch (at most 32 rows in flight per lane)
  static_assert(TB >= 1 && TPW % TB == 0, "whole batches");
  if (vw == 0) return;
  const int lane = lane_id();
  const int wave = wave_in_block();
  const int64_t blk = s / BS;
  const int64_t cbase = (blk * a.nrows + rb) * ROWB + (s - blk * BS) * ELT;
  const int rows = static_cast<int>(re - rb);
  uint8_t* const lin0 = lin + t0 * a.lin_token_stride + rb * ELT;
  // Descriptors of token k of this wave: a token that does not move gets no
  // records, so its accesses are dropped without a lane mask.
  auto token = [&](int k) { return wave + kWaves * k; };
  auto records = [&](int k) -> int { return ((vw >> (token(k) + 1)) & 1ull) ? 0x7FFFFFFF : 0; };
  auto cdesc = [&](int k) {
    return __builtin_amdgcn_make_buffer_rsrc(cache + readlane64(cbase, token(k) + 1), 0, records(k), 0x00020000);
  };
  auto ldesc = [&](int k) {
    return __builtin_amdgcn_make_buffer_rsrc(lin0 + static_cast<int64_t>(token(k)) * a.lin_token_stride, 0,
                                             records(k), 0x00020000);
  };
  // Row r = block * 64 + lane of the group; rows past its end are dropped.
  auto off = [&](int rbk, int bytes) -> uint32_t {
    const int r = rbk * kWave + lane;
    return r < rows ? static_cast<uint32_t>(r * bytes) : kOffOob;
  };
#pragma unroll
  for (int k0 = 0; k0 < TPW; k0 += TB) {
    uint32_t v[TB][NRB];
    // Linear rows: non-temporal (whole lines per instruction); cache columns:
    // default policy (the L2 merges a line's columns).
    constexpr int kSrcBytes = SCATTER ? ELT : ROWB, kSrcPol = SCATTER ? kBufNT : 0;
    constexpr int kDstBytes = SCATTER ? ROWB : ELT, kDstPol = SCATTER ? 0 : kBufNT;
#pragma unroll
    for (int k = 0; k < TB; ++k) {
      const buf_t src = SCATTER ? ldesc(k0 + k) : cdesc(k0 + k);
#pragma unroll
      for (int q = 0; q < NRB; ++q) {
        if constexpr (ELT == 2) v[k][q] = __builtin_amdgcn_raw_buffer_load_b16(src, off(q, kSrcBytes), 0, kSrcPol);
        else v[k][q] = __builtin_amdgcn_raw_buffer_load_b32(src, off(q, kSrcBytes), 0, kSrcPol);
      }
    }
#pragma unroll
    for (int k = 0; k < TB; ++k) {
      const buf_t dst = SCATTER ? cdesc(k0 + k) : ldesc(k0 + k);
#pragma unroll
      for (int q = 0; q < NRB; ++q) {
        if constexpr (ELT == 2)
          __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(v[k][q]), dst, off(q, kDstBytes), 0, kDstPol);
        else
          __builtin_amdgcn_raw_buffer_store_b32(v[k][q], dst, off(q, kDstBytes), 0, kDstPol);
      }
    }
  }
}

// Scatter runs of a tile that average fewer than this many tokens take
// token_rows.  Measured against one 16-bit layer ([8192, 8, 128, 16] cache,
// 16-4,096 tokens in runs of k): k = 1-4 faster (4,096 tokens of runs of 3:
// 45.2 -> 41.0 us; 256 tokens of single tokens 37.2 -> 11.6 us), k = 6 level
// (31.9 against 32.5 us).
constexpr int kShortRunTokens = 6;

// Gathers take token_rows only in launches of at most kTokenGatherTokens
// tokens (a kernel instantiation of their own, TOKG): compiled into every
// gather, the form cost configs[0]'s gather 4 % (5,030 -> 4,860 GB/s) though
// none of its tiles took it.  There a tile takes it when its runs average
// fewer than kShortGatherRunTokens tokens and none goes on past the tile.
constexpr int64_t kTokenGatherTokens = 256;
constexpr int kShortGatherRunTokens = 3;

// Waves per SIMD the tile kernel's register budget must allow: all eight
// (64 VGPRs), which the short-launch scatters over 16- and 32-column blocks
// otherwise miss by 7 registers; 8-column scatters would spill, and keep the
// compiler's choice (at least one wave).
template <int BS, bool SCATTER>
constexpr int kTileMinWaves = (SCATTER && BS == 8) ? 1 : 8;

// FEW selects the form for launches bound by per-workgroup latency rather than
// by HBM: for a scatter the loads-first chunk loop, for a gather the natural
// workgroup order (FEW false: the XCD-contiguous order).  NT is the workgroup
// size; a chunk is NT 16-byte pieces.  LSTP: cache-policy bits of a gather's
// linear-side stores.
template <int ELT, int BS, bool SCATTER, bool FEW, int NT = kCoopThreads, int LSTP = kBufNT, bool TOKG = false>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(kTileMinWaves<BS, SCATTER>)))
void paged_tile_kernel(const TileArgs a) {
  using S = CoopShape<ELT, BS, NT>;
  constexpr int CG = S::CG, NCG = S::NCG, ROWB = S::ROWB, kRows = S::kRows;
  constexpr int RPL = S::RPL, PITCH = S::PITCH;
  static_assert(kTileTokens + BS + 1 <= kWave, "run window must fit one wave");
  __shared__ __align__(16) uint8_t tile[kRows * PITCH];

  const int tid = static_cast<int>(threadIdx.x);
  const int lane = lane_id();
  // Grid: a scatter runs (tile, plane, row group) as (x, y, z); a gather puts
  // the row groups of one tile next to each other in x, so the pieces of one
  // cache block are read by neighbouring workgroups at the same time (3 %
  // faster on random blocks than visiting each group of all tiles in turn).
  // Gathers over many planes give each XCD a contiguous eighth of the grid
  // (FEW false; chosen by the launcher).
  const WgXyz wg = xcd_contiguous_wg<!SCATTER && !FEW>();
  const int64_t tile_id = SCATTER ? static_cast<int64_t>(wg.x) : static_cast<int64_t>(wg.x) / a.row_groups;
  const int64_t group =
      SCATTER ? static_cast<int64_t>(wg.z) : static_cast<int64_t>(wg.x) - tile_id * a.row_groups;
  const int64_t t0 = tile_id * kTileTokens;
  if (t0 >= a.num_tokens) return;
  const int plane = static_cast<int>(wg.y);
  const int layer = plane >> 1;
  const int kv = plane & 1;
  // Rows [rb, re) of the block, in chunks of kRows.
  constexpr int kGroupRows = kRows * kChunksPerGroup<SCATTER>;
  const int64_t rb = group * kGroupRows;
  const int64_t re = (rb + kGroupRows < a.nrows) ? rb + kGroupRows : a.nrows;
  const int nchunks = static_cast<int>((re - rb + kRows - 1) / kRows);
  uint8_t* const cache = a.cache[kv] + static_cast<int64_t>(layer) * a.cache_layer_stride;
  uint8_t* const lin = a.lin[kv] + static_cast<int64_t>(layer) * a.lin_layer_stride;

  // Slot window, identical in every wave: lane i holds token t0 - 1 + i.
  const int64_t t = t0 - 1 + lane;
  int64_t s = -1;
  if (t >= 0 && t < a.num_tokens) s = slot_at(a, t);
  bool valid = (s >= 0) && (s < a.num_slots);
  if constexpr (SCATTER) {
    if (a.scan_dupes) {
      ScanTable& scan = scan_table();
      scan_build<NT>(scan, a);
      if (valid) valid = scan_is_last(scan, s, t);
    } else if (valid && a.owner != nullptr) {
      valid = (a.owner[s] == claim_tag(a.epoch, t));
    }
  }
  const uint64_t vmask = ballot(valid);
  const int64_t s_prev = from_prev_lane(s);
  const bool prev_valid = lane > 0 && ((vmask >> (lane - 1)) & 1ull);
  const bool cont = valid && prev_valid && (s == s_prev + 1) && ((s % BS) != 0);
  const uint64_t cmask = ballot(cont);
  const int64_t remaining = a.num_tokens - t0;
  const int ntile = remaining < kTileTokens ? static_cast<int>(remaining) : kTileTokens;
  const uint64_t window = ((1ull << ntile) - 1ull) << 1;
  uint64_t heads = vmask & ~cmask & window;

  // This thread's cache piece (row pr, column group pg) and linear piece
  // (block column lc, row group lq) within every chunk.  All offsets are
  // 32-bit and relative to the run's descriptors; per chunk they advance by a
  // constant.
  const int pr = tid / NCG;
  const int pg = tid % NCG;
  const int rows_left = static_cast<int>(re - rb);
  const int lc = S::col(tid);
  const int lq = S::grp(tid);
  auto prow_in = [&](int k) { return k * kRows + pr < rows_left; };
  auto lrow_in = [&](int k) { return k * kRows + lq * RPL < rows_left; };
  constexpr uint32_t kCacheStep = kRows * ROWB;     // bytes between chunks, cache side
  constexpr uint32_t kLinStep = kRows * ELT;        // bytes between chunks, linear side
  const uint32_t cpiece = static_cast<uint32_t>(tid) * 16u;
  const uint32_t stride32 = static_cast<uint32_t>(a.lin_token_stride);

  if constexpr (SCATTER) {
    // Lanes of the runs that start in this tile (lanes at its start that
    // continue an earlier tile's run belong to that tile): adding a head's
    // next bit to cmask carries through exactly the continuation bits of its
    // run.  The tile's last run may go on past the tile's end and keeps the
    // run form; short runs before it move with token_rows.
    uint64_t tok_heads = heads;
    uint64_t tok_lanes = heads | (((cmask + (heads << 1)) ^ cmask) & cmask);
    if (tok_lanes & ~window) {
      const uint64_t below_last = (1ull << (63 - __builtin_clzll(heads))) - 1ull;
      tok_heads &= below_last;
      tok_lanes &= below_last;
    }
    const int truns = __builtin_popcountll(tok_heads);
    if (truns > 0 && __builtin_popcountll(tok_lanes) < truns * kShortRunTokens) {
      token_rows<ELT, BS, NT, true>(a, cache, lin, s, tok_lanes, t0, rb, re);
      heads &= ~tok_heads;
    }
  }
  if constexpr (!SCATTER && TOKG) {
    // The same lanes for a gather, which takes token_rows only for a whole
    // tile (all its runs, none of them going on past the tile).
    const uint64_t owned = heads | (((cmask + (heads << 1)) ^ cmask) & cmask);
    const int nr = __builtin_popcountll(heads);
    if (nr > 0 && (owned & ~window) == 0 && __builtin_popcountll(owned) < nr * kShortGatherRunTokens) {
      token_rows<ELT, BS, NT, false>(a, cache, lin, s, owned, t0, rb, re);
      heads = 0;
    }
  }

  [[maybe_unused]] bool tile_used = false;  // wave-uniform: some chunk of this workgroup has filled the LDS tile
  while (heads) {
    const int i = __builtin_ctzll(heads);
    heads &= heads - 1;
    const uint64_t after = cmask >> (i + 1);  // i <= kTileTokens < 63
    const int len = 1 + __builtin_ctzll(~after);
    const int64_t sh = readlane64(s, i);
    const int64_t blk = sh / BS;
    const int c0 = static_cast<int>(sh - blk * BS);
    const int c1 = c0 + len;
    const int64_t tf = t0 - 1 + i;
    // Wave-uniform descriptors: the block's rows [rb, re) and the run's
    // first linear row at row rb.  Offsets of masked lanes are kOffOob.
    const buf_t cbuf = make_buf(cache + (blk * a.nrows + rb) * ROWB);
    const buf_t lbuf = make_buf(lin + tf * a.lin_token_stride + rb * ELT);
    const bool lmine = lc >= c0 && lc < c1;
    const uint32_t lbase = static_cast<uint32_t>(lc - c0) * stride32 + static_cast<uint32_t>(lq) * 16u;
    auto coff = [&](int k) -> uint32_t { return prow_in(k) ? cpiece + k * kCacheStep : kOffOob; };
    auto loff = [&](int k) -> uint32_t { return (lmine && lrow_in(k)) ? lbase + k * kLinStep : kOffOob; };

    // Every payload load of the run is issued before its first store.  Wave
    // memory counters retire in issue order, so a wait for a load issued after
    // a store would also wait for that store's round trip.
    constexpr int C = kChunksPerGroup<SCATTER>;
    if constexpr (!SCATTER) {
      u32x4 v[C];
#pragma unroll
      for (int k = 0; k < C; ++k) v[k] = buf_ld16(cbuf, k < nchunks ? coff(k) : kOffOob);
#pragma unroll
      for (int k = 0; k < C; ++k) {
        if (k >= nchunks) break;
        if (tile_used) lds_barrier();  // the tile's previous column reads are done
        tile_used = true;
        if (prow_in(k)) {
          uint32_t* const d = reinterpret_cast<uint32_t*>(tile + pr * PITCH + pg * 16);
          d[0] = v[k][0]; d[1] = v[k][1]; d[2] = v[k][2]; d[3] = v[k][3];
        }
        lds_barrier();
        buf_st16_p<LSTP>(lbuf, loff(k), lds_column_piece<ELT, PITCH>(tile, lq * RPL, lc));
      }
    } else if constexpr (!FEW) {
      scatter_run_chunks<ELT, BS, NT>(tile, cbuf, lbuf, c0, c1, nchunks, rows_left, stride32);
    } else {
      // Small scatters (a few rounds of workgroups) are bound by each
      // workgroup's latency.  Full and partial runs are separate straight-line
      // paths, so that the compiler's wait counts are exact on each and no
      // chunk's load wait covers an earlier chunk's stores.
      auto scatter_run = [&](auto full_tag) {
        constexpr bool kFull = decltype(full_tag)::value;
        u32x4 v[C];
#pragma unroll
        for (int k = 0; k < C; ++k) v[k] = buf_ld16(lbuf, k < nchunks ? loff(k) : kOffOob);
#pragma unroll
        for (int k = 0; k < C; ++k) {
          if (k >= nchunks) break;
          if (tile_used) lds_barrier();  // the tile's previous row reads are done
          tile_used = true;
          if (lmine && lrow_in(k)) lds_put_column<ELT, PITCH>(tile, lq * RPL, lc, v[k]);
          lds_barrier();
          const uint32_t* const d = reinterpret_cast<const uint32_t*>(tile + pr * PITCH + pg * 16);
          const u32x4 w = {d[0], d[1], d[2], d[3]};
          const uint32_t off = coff(k);
          if constexpr (kFull) {
            buf_st16(cbuf, off, w);
          } else {
            // Whole pieces inside the run go as one vector; edge pieces store
            // only their in-run columns.
            const int lo = pg * CG;
            const bool whole = lo >= c0 && lo + CG <= c1;
            buf_st16(cbuf, whole ? off : kOffOob, w);
#pragma unroll
            for (int cc = 0; cc < CG; ++cc) {
              const bool mine = !whole && off != kOffOob && lo + cc >= c0 && lo + cc < c1;
              buf_st_elem<ELT>(cbuf, mine ? off + cc * ELT : kOffOob, piece_elem<ELT>(w, cc));
            }
          }
        }
      };
      if (c0 == 0 && c1 == BS) scatter_run(std::true_type{});
      else scatter_run(std::false_type{});
    }
  }

  if constexpr (!SCATTER) {
    if (a.fill_zeros) {
      // Skipped tokens (the positions past seq_lens of a dense preload, a
      // negative slot) get zero rows.  All threads share the work: thread tid
      // writes piece tid % P of the (tid / P)-th skipped token of each pass,
      // P being the 16-byte pieces of one token's row group.
      const uint64_t skipped = ~vmask & window;
      constexpr int P = kRows * kChunksPerGroup<false> * ELT / 16;
      static_assert(NT % P == 0, "a pass covers whole tokens");
      constexpr int kTokensPerPass = NT / P;
      const int64_t k = rb * ELT + static_cast<int64_t>(tid % P) * 16;
      const int nskip = __builtin_popcountll(skipped);
      const u32x4 zero = {0u, 0u, 0u, 0u};
      for (int o = tid / P; o < nskip; o += kTokensPerPass) {
        uint64_t m = skipped;
        for (int j = 0; j < o; ++j) m &= m - 1;  // drop the first o skipped tokens
        const int i = __builtin_ctzll(m);
        if (k < re * ELT) st16(lin + (t0 - 1 + i) * a.lin_token_stride + k, zero);
      }
    }
  }
}

// ----- block-major scatter ------------------------------------------------------
//
// The scatter visited in destination order.  Its claim pass has recorded, for
// every destination slot, the last token that writes it (tag = epoch << 32 |
// token + 1, with an epoch no earlier call on the array used), so the scatter
// can run as a gather over that inverse map: one workgroup per (cache block,
// plane, row group) in block order reads its BS tags, finds the runs of
// consecutive tokens in consecutive slots, and copies each run like the
// token-major kernel.  Cache blocks are then written in address order and the
// linear rows read in slot order: on configs[1]'s buffers the block-pattern
// copy moves the scatter's bytes at 6.19 TB/s this way against 5.80 TB/s
// with the cache blocks written in token order (random writes cost more than
// random reads on this GPU).  Blocks no token writes cost one tag read.
constexpr int kBlockScatterChunks = 2;  // chunks per workgroup of the block-major scatter

// Grid: x = block * row_groups + group (the row groups of one block next to
// each other), y = plane.  XCD: each XCD takes a contiguous eighth of the
// grid (a range of planes) instead of every eighth workgroup.
template <int ELT, int BS, bool XCD, int CSTP = kBufNT, int NT = kCoopThreads>
__global__ __launch_bounds__(NT) void paged_block_scatter_kernel(const TileArgs a) {
  using S = CoopShape<ELT, BS, NT>;
  constexpr int ROWB = S::ROWB, kRows = S::kRows;
  static_assert(BS <= kWave, "one lane per slot of a block");
  __shared__ __align__(16) uint8_t tile[kRows * S::PITCH];

  const int lane = lane_id();
  const uint32_t g = static_cast<uint32_t>(a.row_groups);
  const WgXyz wg = xcd_contiguous_wg<XCD>();
  const uint32_t bq = wg.x / g;
  const int64_t blk = bq;
  const int64_t grp = wg.x - bq * g;
  const int plane = static_cast<int>(wg.y);
  const int layer = plane >> 1;
  const int kv = plane & 1;
  constexpr int kGroupRows = kRows * kBlockScatterChunks;
  const int64_t rb = grp * kGroupRows;
  const int64_t re = (rb + kGroupRows < a.nrows) ? rb + kGroupRows : a.nrows;
  const int nchunks = static_cast<int>((re - rb + kRows - 1) / kRows);

  // Lane p < BS holds the tag of slot blk * BS + p.
  uint64_t tag = 0;
  if (lane < BS) tag = a.owner[blk * BS + lane];
  const bool valid = lane < BS && static_cast<uint32_t>(tag >> 32) == a.epoch && static_cast<uint32_t>(tag) != 0u;
  const int64_t tok = static_cast<int64_t>(static_cast<uint32_t>(tag)) - 1;
  const uint64_t vmask = ballot(valid);
  if (vmask == 0) return;
  const int64_t tok_prev = from_prev_lane(tok);
  const bool prev_valid = lane > 0 && ((vmask >> (lane - 1)) & 1ull);
  const uint64_t cmask = ballot(valid && prev_valid && tok == tok_prev + 1);
  uint64_t heads = vmask & ~cmask;

  uint8_t* const cache = a.cache[kv] + static_cast<int64_t>(layer) * a.cache_layer_stride;
  const uint8_t* const lin = a.lin[kv] + static_cast<int64_t>(layer) * a.lin_layer_stride;
  const buf_t cbuf = make_buf(cache + (blk * a.nrows + rb) * ROWB);
  const uint32_t stride32 = static_cast<uint32_t>(a.lin_token_stride);
  while (heads) {
    const int c0 = __builtin_ctzll(heads);
    heads &= heads - 1;
    const int len = 1 + __builtin_ctzll(~(cmask >> (c0 + 1)));  // c0 < BS <= 32
    const int64_t tf = readlane64(tok, c0);
    const buf_t lbuf = make_buf(lin + tf * a.lin_token_stride + rb * ELT);
    scatter_run_chunks<ELT, BS, NT, CSTP>(tile, cbuf, lbuf, c0, c0 + len, nchunks, static_cast<int>(re - rb),
                                          stride32);
  }
}

// ----- generic element-wise kernel (any block size / alignment) ----------------

template <int ELT_C, int ELT_L, int CODEC, int LDT, bool SCATTER>
__global__ __launch_bounds__(kBlockThreads) void paged_elem_kernel(const TileArgs a) {
  const int plane = static_cast<int>(blockIdx.y);
  const int layer = plane >> 1;
  const int kv = plane & 1;
  uint8_t* const cache = a.cache[kv] + static_cast<int64_t>(layer) * a.cache_layer_stride;
  uint8_t* const lin = a.lin[kv] + static_cast<int64_t>(layer) * a.lin_layer_stride;
  const int64_t total = a.num_tokens * a.nrows;
  const int64_t bs = a.block_size;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < total;
       e += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t t = e / a.nrows;
    const int64_t r = e - t * a.nrows;
    const int64_t s = slot_at(a, t);
    bool valid = (s >= 0) && (s < a.num_slots);
    if constexpr (SCATTER) {
      if (valid && a.owner != nullptr) valid = (a.owner[s] == claim_tag(a.epoch, t));
    }
    uint8_t* const lp = lin + t * a.lin_token_stride + r * ELT_L;
    if (!valid) {
      if (!SCATTER && a.fill_zeros) store_elem<ELT_L>(lp, 0u);
      continue;
    }
    const int64_t blk = s / bs;
    const int64_t off = s - blk * bs;
    uint8_t* const cp = cache + ((blk * a.nrows + r) * bs + off) * ELT_C;
    float sc = 1.0f;
    if constexpr (CODEC != kCopy) sc = load_scale(a, kv, layer, r / a.head_dim);
    if constexpr (!SCATTER) {
      uint32_t v = load_elem<ELT_C>(cp);
      if constexpr (CODEC != kCopy) v = f32_to_lin<LDT>(fp8_decode<CODEC>(v) * sc);
      store_elem<ELT_L>(lp, v);
    } else {
      uint32_t v = load_elem<ELT_L>(lp);
      if constexpr (CODEC != kCopy) v = fp8_encode<CODEC>(div_rn(lin_to_f32<LDT>(v), sc));
      store_elem<ELT_C>(cp, v);
    }
  }
}

// ----- host dispatch --------------------------------------------------------------

namespace {

template <int ELT_C, int ELT_L, int CODEC, int LDT, bool SCATTER>
hipError_t launch_elem(const TileArgs& a, int64_t planes, hipStream_t stream) {
  const int64_t total = a.num_tokens * a.nrows;
  int64_t blocks = (total + kBlockThreads - 1) / kBlockThreads;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL((paged_elem_kernel<ELT_C, ELT_L, CODEC, LDT, SCATTER>),
                     dim3(static_cast<uint32_t>(blocks), static_cast<uint32_t>(planes)), dim3(kBlockThreads), 0,
                     stream, a);
  return hipGetLastError();
}

// Scatters of at most this many workgroups (about four rounds of resident
// workgroups on 256 CUs) take the loads-first chunk loop (FEW true).
constexpr int64_t kFewGroups = 8192;
// Gathers over at least this many planes take the XCD-contiguous workgroup
// order (FEW false).  Measured on 128,708 tokens: the natural order slows
// from 6.14 TB/s at 2 planes to 5.77 TB/s at 64, the XCD-contiguous order
// stays at 5.88-5.92 TB/s; they cross between 16 and 32 planes.  Short
// launches keep the natural order too (cfg 1: 13.0 against 13.9 us).
constexpr int64_t kXcdOrderPlanes = 32;

// 16-bit gathers whose 256-thread grid has at most kFewGroups workgroups use
// 128-thread workgroups (2 KiB chunks) for block sizes up to 16.  Measured on
// 1-4 planes of short sequences: 3-4 % faster with skipped slots or several
// layers (4 bf16 layers: 13.5 -> 12.9 us), unchanged on configs[0] without
// skips (12.9 us), 1 % slower for fp32 (chunks of only 32 rows).
constexpr int kShortGatherThreads = 128;

// Tile grid of one launch with NT-thread workgroups: (tile, plane, row group)
// for a scatter, (tile x row group, plane) for a gather.
template <int ELT, int BS, bool SCATTER, int NT>
hipError_t tile_grid(const TileArgs& a0, int64_t planes, TileArgs* a, dim3* grid, int64_t* workgroups) {
  using S = CoopShape<ELT, BS, NT>;
  constexpr int kGroupRows = S::kRows * kChunksPerGroup<SCATTER>;
  const int64_t groups = (a0.nrows + kGroupRows - 1) / kGroupRows;
  if (groups > 65535) return hipErrorInvalidValue;
  const int64_t tiles = (a0.num_tokens + kTileTokens - 1) / kTileTokens;
  *a = a0;
  a->row_groups = static_cast<int32_t>(groups);
  if constexpr (SCATTER) {
    if (tiles > 0x7FFFFFFF) return hipErrorInvalidValue;
    *grid = dim3(static_cast<uint32_t>(tiles), static_cast<uint32_t>(planes), static_cast<uint32_t>(groups));
  } else {
    if (tiles > 0x7FFFFFFF / groups) return hipErrorInvalidValue;
    *grid = dim3(static_cast<uint32_t>(tiles * groups), static_cast<uint32_t>(planes), 1);
  }
  *workgroups = tiles * planes * groups;
  return hipSuccess;
}

// True when every linear token row of the launch covers whole 128-byte lines
// (row size, token and layer strides, both bases): only then do write-through
// stores leave no line to be written once per token.
bool linear_rows_whole_lines(const TileArgs& a, int elt) {
  constexpr int64_t kLine = 128;
  return (a.nrows * elt) % kLine == 0 && a.lin_token_stride % kLine == 0 && a.lin_layer_stride % kLine == 0 &&
         reinterpret_cast<uintptr_t>(a.lin[0]) % kLine == 0 && reinterpret_cast<uintptr_t>(a.lin[1]) % kLine == 0;
}

template <int ELT, int BS, bool SCATTER>
hipError_t launch_tile(const TileArgs& a0, int64_t planes, hipStream_t stream) {
  if constexpr (SCATTER) {
    // Destination order when the claim tags form this call's inverse map and
    // the tokens cover a good share of the cache's slots (each block of the
    // cache costs a workgroup that reads its tags).
    if (a0.owner != nullptr && a0.owner_exclusive && a0.num_tokens * 4 >= a0.num_slots &&
        a0.num_slots / BS <= 0x7FFFFFFF && a0.num_slots % BS == 0) {
      // Two 4 KiB chunks per workgroup, and the four workgroups of a block
      // next to each other in the grid (x = block * groups + group): on the
      // configs[1] scatter 5.60 TB/s, against 5.46-5.52 with four chunks (grid
      // z or folded), 5.33 with eight and 4.80 with one.
      // 16-bit launches over fewer planes than the XCD order wants take the
      // per-wave kernel (a workgroup per block, no workgroup barrier): the
      // dense write-back (2 planes) 5.50-5.58 -> 5.60-5.74 TB/s; over
      // configs[1]'s 64 planes the two kernels measured level, and the
      // cooperative one below keeps them.
      if constexpr (ELT == 2) {
        if (planes < kXcdOrderPlanes) return launch_wave_copy_scatter<BS>(a0, planes, stream);
      }
      using S = CoopShape<ELT, BS, kCoopThreads>;
      constexpr int64_t kGroupRows = S::kRows * kBlockScatterChunks;
      const int64_t groups = (a0.nrows + kGroupRows - 1) / kGroupRows;
      const int64_t nblk = a0.num_slots / BS;
      if (nblk * groups <= 0x7FFFFFFF) {
        TileArgs a = a0;
        a.row_groups = static_cast<int32_t>(groups);
        // Whole blocks are written through the L2 (kBufWT): +1.1 % on the
        // configs[1] scatter.  Launches over at least 32 planes give each XCD
        // a contiguous range of planes: configs[1]'s scatter 5.65 -> 5.85
        // TB/s (same buffers, three allocations), where a plane-fastest order
        // ran at 5.46 and non-temporal stores at 5.60; with 2 planes (the
        // dense write-back) the two orders are within noise.
        const dim3 grid(static_cast<uint32_t>(nblk * groups), static_cast<uint32_t>(planes), 1);
        if (planes >= kXcdOrderPlanes)
          hipLaunchKernelGGL((paged_block_scatter_kernel<ELT, BS, true, kBufWT>), grid, dim3(kCoopThreads), 0,
                             stream, a);
        else
          hipLaunchKernelGGL((paged_block_scatter_kernel<ELT, BS, false, kBufWT>), grid, dim3(kCoopThreads), 0,
                             stream, a);
        return hipGetLastError();
      }
    }
  }
  TileArgs a;
  dim3 grid;
  int64_t workgroups = 0;
  hipError_t err = tile_grid<ELT, BS, SCATTER, kCoopThreads>(a0, planes, &a, &grid, &workgroups);
  if (err != hipSuccess) return err;
  const bool lines = !SCATTER && linear_rows_whole_lines(a0, ELT);
  if constexpr (!SCATTER && ELT == 2 && BS <= 16) {
    if (workgroups <= kFewGroups) {
      // Short gathers: twice the workgroups, half the size each (on cfg 2's
      // 64 planes this form is 1 % slower than 256 threads).
      err = tile_grid<ELT, BS, SCATTER, kShortGatherThreads>(a0, planes, &a, &grid, &workgroups);
      if (err != hipSuccess) return err;
      const bool tok = a0.num_tokens <= kTokenGatherTokens;
      if (lines && tok)
        hipLaunchKernelGGL((paged_tile_kernel<ELT, BS, SCATTER, true, kShortGatherThreads, kBufWT, true>), grid,
                           dim3(kShortGatherThreads), 0, stream, a);
      else if (lines)
        hipLaunchKernelGGL((paged_tile_kernel<ELT, BS, SCATTER, true, kShortGatherThreads, kBufWT>), grid,
                           dim3(kShortGatherThreads), 0, stream, a);
      else if (tok)
        hipLaunchKernelGGL((paged_tile_kernel<ELT, BS, SCATTER, true, kShortGatherThreads, kBufNT, true>), grid,
                           dim3(kShortGatherThreads), 0, stream, a);
      else
        hipLaunchKernelGGL((paged_tile_kernel<ELT, BS, SCATTER, true, kShortGatherThreads>), grid,
                           dim3(kShortGatherThreads), 0, stream, a);
      return hipGetLastError();
    }
  }
  // (The XCD order indexes the grid in 32 bits.)  Short and XCD-ordered
  // gathers write linear rows of whole lines through the L2 (kBufWT); the
  // other gathers (few planes, many workgroups: the dense preload) measured
  // no faster with it.
  const bool few = SCATTER ? workgroups <= kFewGroups
                           : !(planes >= kXcdOrderPlanes && workgroups > kFewGroups &&
                               workgroups <= int64_t{0xFFFFFFFF});
  if (few && !SCATTER && a0.num_tokens <= kTokenGatherTokens)
    hipLaunchKernelGGL((paged_tile_kernel<ELT, BS, SCATTER, true, kCoopThreads, kBufNT, !SCATTER>), grid,
                       dim3(kCoopThreads), 0, stream, a);
  else if (few)
    hipLaunchKernelGGL((paged_tile_kernel<ELT, BS, SCATTER, true>), grid, dim3(kCoopThreads), 0, stream, a);
  else if (lines)
    hipLaunchKernelGGL((paged_tile_kernel<ELT, BS, SCATTER, false, kCoopThreads, kBufWT>), grid, dim3(kCoopThreads),
                       0, stream, a);
  else
    hipLaunchKernelGGL((paged_tile_kernel<ELT, BS, SCATTER, false>), grid, dim3(kCoopThreads), 0, stream, a);
  return hipGetLastError();
}

template <int ELT_C, int ELT_L, int CODEC, int LDT, bool SCATTER>
hipError_t dispatch_bs(const TileArgs& a, int64_t bs, bool fast, int64_t planes, hipStream_t stream) {
  if (fast) {
    if constexpr (CODEC == kCopy) {
      // 16- and 32-bit copies: workgroup-cooperative kernel.
      static_assert(ELT_C == ELT_L, "copies keep the element type");
      if (bs == 8) return launch_tile<ELT_C, 8, SCATTER>(a, planes, stream);
      if (bs == 16) return launch_tile<ELT_C, 16, SCATTER>(a, planes, stream);
      if (bs == 32) return launch_tile<ELT_C, 32, SCATTER>(a, planes, stream);
    } else if constexpr (!SCATTER) {
      // FP8 dequant-gather: per-wave kernel (kv_paged_waves.hip), unless a chunk
      // of its rows spans more heads than its decode tables hold.
      hipError_t err = hipErrorNotSupported;
      if (bs == 16) err = launch_wave_gather<ELT_C, ELT_L, CODEC, LDT, 16>(a, planes, stream);
      if (bs == 32) err = launch_wave_gather<ELT_C, ELT_L, CODEC, LDT, 32>(a, planes, stream);
      if (err != hipErrorNotSupported) return err;
    } else {
      // FP8 quant-store: per-wave kernel (kv_paged_waves.hip).
      if (bs == 16) return launch_wave_scatter<ELT_C, ELT_L, CODEC, LDT, 16>(a, planes, stream);
      if (bs == 32) return launch_wave_scatter<ELT_C, ELT_L, CODEC, LDT, 32>(a, planes, stream);
    }
  }
  // The element kernel checks claim tags only: a call without them takes the
  // claim pass first.
  if (SCATTER && a.scan_dupes) return hipErrorNotSupported;
  return launch_elem<ELT_C, ELT_L, CODEC, LDT, SCATTER>(a, planes, stream);
}

template <int ELT_C, int ELT_L, int CODEC, int LDT>
hipError_t dispatch_dir(const TileArgs& a, const PagedTileParams& p, bool fast, int64_t planes, hipStream_t stream) {
  if (p.scatter) return dispatch_bs<ELT_C, ELT_L, CODEC, LDT, true>(a, p.block_size, fast, planes, stream);
  return dispatch_bs<ELT_C, ELT_L, CODEC, LDT, false>(a, p.block_size, fast, planes, stream);
}

template <int CODEC>
hipError_t dispatch_fp8(const TileArgs& a, const PagedTileParams& p, bool fast, int64_t planes, hipStream_t stream) {
  switch (p.lin_dtype) {
    case kLinBF16: return dispatch_dir<1, 2, CODEC, kLinBF16>(a, p, fast, planes, stream);
    case kLinF16: return dispatch_dir<1, 2, CODEC, kLinF16>(a, p, fast, planes, stream);
    case kLinF32: return dispatch_dir<1, 4, CODEC, kLinF32>(a, p, fast, planes, stream);
    default: return hipErrorInvalidValue;
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t launch_paged_tiles(const PagedTileParams& p, hipStream_t stream) {
  if (p.num_tokens <= 0 || p.num_layers <= 0) return hipSuccess;
  if (p.num_blocks <= 0 || p.num_heads <= 0 || p.head_dim <= 0 || p.block_size <= 0) return hipErrorInvalidValue;
  if (p.num_layers * 2 > 65535) return hipErrorInvalidValue;
  const bool fp8 = p.codec != kCopy;
  if (fp8 ? (p.cache_elt != 1 || (p.lin_elt != 2 && p.lin_elt != 4))
          : ((p.cache_elt != 2 && p.cache_elt != 4) || p.lin_elt != p.cache_elt))
    return hipErrorInvalidValue;
  if (fp8 && p.scale[0] == nullptr) return hipErrorInvalidValue;

  TileArgs a{};
  for (int i = 0; i < 2; ++i) {
    a.cache[i] = static_cast<uint8_t*>(p.cache[i]);
    a.lin[i] = static_cast<uint8_t*>(p.lin[i]);
    a.scale[i] = p.scale[i] ? p.scale[i] : p.scale[0];
  }
  a.slots = p.slots;
  a.owner = p.owner;
  a.num_tokens = p.num_tokens;
  a.num_slots = p.num_blocks * p.block_size;
  a.nrows = p.num_heads * p.head_dim;
  a.head_dim = p.head_dim;
  a.num_heads = p.num_heads;
  a.cache_layer_stride = p.num_blocks * a.nrows * p.block_size * p.cache_elt;
  a.lin_layer_stride = p.lin_layer_stride;
  a.lin_token_stride = p.lin_token_stride;
  a.scale_mode = p.scale_mode;
  a.fill_zeros = p.fill_zeros;
  a.epoch = p.epoch;
  a.owner_exclusive = p.owner_exclusive;
  a.scan_dupes = p.scan_dupes;
  if (a.scan_dupes && (!p.scatter || p.num_tokens > kScanTokens)) return hipErrorInvalidValue;
  a.block_size = static_cast<int32_t>(p.block_size);
  a.inv_head_dim = 1.0f / static_cast<float>(p.head_dim);
  a.bt = p.bt;
  if (a.bt.block_tables != nullptr) {
    // Dense tokens are numbered in 32 bits; block ids and sizes stay 32-bit too.
    if (a.bt.seq_lens == nullptr || a.bt.dense_len == 0 || a.bt.max_blocks < 0 ||
        p.num_tokens >= (int64_t{1} << 31) || p.block_size >= (int64_t{1} << 31))
      return hipErrorInvalidValue;
    a.bt.block_size = static_cast<int32_t>(p.block_size);
    a.bt.num_blocks = p.num_blocks;
  } else if (p.slots == nullptr) {
    return hipErrorInvalidValue;
  }

  const int rpl = 16 / p.lin_elt;
  const int cg = 16 / p.cache_elt;
  // The tile kernels address one run with 32-bit offsets (token stride up to
  // 32 MiB) and divide row numbers below 2^24 by head_dim in float.
  bool fast = (p.head_dim % rpl == 0) && (p.lin_token_stride % 16 == 0) && (p.lin_layer_stride % 16 == 0) &&
              (p.block_size % cg == 0) && (p.lin_token_stride <= (int64_t{1} << 25)) &&
              (a.nrows < (int64_t{1} << 24));
  for (int i = 0; i < 2; ++i) fast = fast && aligned16(a.cache[i]) && aligned16(a.lin[i]);

  const int64_t planes = p.num_layers * 2;
  if (!fp8) {
    if (p.cache_elt == 2) return dispatch_dir<2, 2, kCopy, kLinBF16>(a, p, fast, planes, stream);
    return dispatch_dir<4, 4, kCopy, kLinF32>(a, p, fast, planes, stream);
  }
  if (p.codec == kE4M3) return dispatch_fp8<kE4M3>(a, p, fast, planes, stream);
  if (p.codec == kE5M2) return dispatch_fp8<kE5M2>(a, p, fast, planes, stream);
  return hipErrorInvalidValue;
}

}  // namespace kvhip
