// Per-wave paged-A <-> linear kernels for MI355X (gfx950): the FP8
// dequant-gather and quant-store, and the 16-bit scatter in destination order
// for launches over few planes.
//
// Dequant-gather.  One wave owns the runs (consecutive tokens in consecutive
// slots of one block) that start in its 16-token tile, for one chunk of cache
// rows (grid z).  A chunk is 64 lane tiles of RPL rows x CG block columns:
// each lane loads its own tile, RPL 16-byte pieces of consecutive cache rows
// (cached loads: a wave instruction touches 64 lines partially and the L2
// serves the rest of each line to the next instructions), so the lane holds
// RPL rows x CG tokens and writes 16-byte pieces of token rows.  Each code is
// decoded by one LDS read from the workgroup's decode tables (value x scale
// already rounded to the linear type), about 2.5 VALU instructions per
// element against 16.8 for decoding, scaling and rounding in registers.  The
// LDS holds only those tables (4 KiB); the launch pads it so that 3
// workgroups share a CU (launch_wave_gather).  Copies (no decode) stage the chunk through the wave's LDS
// region instead: coalesced loads, exchanged so that each lane holds its tile.
// Runs that do not cover every column group of the block row load only the
// column groups they cover.
#include "kv_hip_common.h"
#include "kv_launch.h"
#include "kv_paged_args.h"

namespace kvhip {

namespace {

// d[q] holds 16 bytes of cache row (r0+q) for one column group; returns the
// 16-byte linear piece (rows r0..r0+RPL-1) of block column `cc`.  FP8 codes
// are decoded through `lut`, the lane's head's table of 256 linear-side
// values (decode(code) * scale, rounded to the linear type).
template <int ELT_C, int ELT_L, int CODEC, int RPL, typename LutT>
__device__ __forceinline__ u32x4 gather_column(const u32x4 (&d)[RPL], int cc, const LutT* lut) {
  u32x4 o;
  if constexpr (CODEC == kCopy && ELT_C == 2) {
    static_assert(RPL == 8, "16-bit tiles are 8x8");
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = pack16(elem16(d[2 * k], cc), elem16(d[2 * k + 1], cc));
  } else if constexpr (CODEC == kCopy && ELT_C == 4) {
    static_assert(RPL == 4, "fp32 tiles are 4x4");
#pragma unroll
    for (int k = 0; k < 4; ++k) o[k] = d[k][cc];
  } else {
    static_assert(ELT_C == 1, "fp8 caches hold one byte per element");
    if constexpr (ELT_L == 2) {
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = pack16(lut[elem8(d[2 * k], cc)], lut[elem8(d[2 * k + 1], cc)]);
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = lut[elem8(d[k], cc)];
    }
  }
  return o;
}

// Decoded-value tables of the FP8 dequant-gather, built once per workgroup in
// LDS: entry (j, code) holds the linear-side bits of decode(code) * scale of
// head h_lo + j (for a scalar scale, one table), computed by the same scalar
// steps as the per-element decode (fp8_decode, fp32 multiply, f32_to_lin), so
// a lookup returns exactly what decoding the element would.  A chunk spans at
// most kLutHeads heads at the shapes this kernel serves (head_dim >= 64);
// chunks spanning more decode per element.
constexpr int kLutHeads = 8;

template <int ELT_L>
struct LutEntry {
  using T = uint32_t;
};
template <>
struct LutEntry<2> {
  using T = uint16_t;
};

template <int CODEC, int LDT, typename T>
__device__ __forceinline__ T lut_value(uint32_t code, float sc) {
  return static_cast<T>(f32_to_lin<LDT>(fp8_decode<CODEC>(code) * sc));
}

// Piece s of a chunk lives at LDS slot lds_slot(s): the low four bits are
// XOR-swizzled with the row group so that 16 consecutive lanes hit 16
// distinct 16-byte bank groups both when lanes take consecutive pieces and
// when each lane takes the RPL pieces of its tile.
constexpr int log2_const(int v) { return v <= 1 ? 0 : 1 + log2_const(v / 2); }

template <int RPL, int NCG>
__device__ __forceinline__ int lds_slot(int s) {
  constexpr int kGroupShift = log2_const(RPL * NCG);
  return s ^ (((s >> kGroupShift) * NCG) & 15);
}

// Orders the wave's LDS writes before its later LDS reads (and the reads
// before the next writes).  LDS executes one wave's requests in issue order;
// the wait plus the code-motion barrier keep the compiler from reordering.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), other counters untouched
  __builtin_amdgcn_wave_barrier();
}

template <int ELT_C, int ELT_L, int BS>
struct WaveShape {
  static constexpr int RPL = 16 / ELT_L;             // cache rows per lane tile
  static constexpr int CG = 16 / ELT_C;              // block columns per 16-byte group
  static constexpr int NCG = BS / CG;                // 16-byte groups per cache row
  static constexpr int kChunkRows = (kWave / NCG) * RPL;
  static_assert(BS % CG == 0, "block row must be a whole number of 16-byte groups");
};

// STP: cache-policy bits of the full runs' linear stores (kBufWT when every
// linear row is whole 128-byte lines).
// Dequant-gather tiles of short runs in small launches (TOKG: a kernel
// instantiation of its own, for calls of at most kTokenGatherTokens tokens):
// instead of walking the runs one by one, the wave moves its chunk's rows of
// every such token at once, one row per lane (row r0 + m * 64 + lane, M =
// kChunkRows / 64 rows per token): the token's code byte through a scalar
// buffer descriptor of its block column (no records for a token that does
// not move), its value from the head's decode table, and the element to the
// token's linear row.  `lut_off[m]` is the offset of row m's table.  Lane
// i + 1 of `s` holds the slot of token t0 + i; bit i + 1 of `vw` says that the
// token moves.
template <int ELT_L, int BS, int M, typename LutT>
__device__ __forceinline__ void dequant_token_rows(const TileArgs& a, const uint8_t* cache, uint8_t* lin,
                                                   const LutT* lut_all, const int (&lut_off)[M], int64_t s,
                                                   uint64_t vw, int64_t t0, int64_t r0, int64_t r_end) {
  constexpr int TB = 32 / M < kTileTokens ? 32 / M : kTileTokens;  // tokens per batch: 32 codes in flight per lane
  static_assert(kTileTokens % TB == 0, "whole batches");
  int lane = lane_id();
  asm volatile("" : "+v"(lane));
  const int64_t blk = s / BS;
  const int64_t cbase = (blk * a.nrows + r0) * BS + (s - blk * BS);
  uint8_t* const lin0 = lin + t0 * a.lin_token_stride + r0 * ELT_L;
  const int rows = static_cast<int>(r_end - r0);
  auto off = [&](int m, int bytes) -> uint32_t {
    return m * kWave + lane < rows ? static_cast<uint32_t>((m * kWave + lane) * bytes) : kOffOob;
  };
  auto records = [&](int i) -> int { return ((vw >> (i + 1)) & 1ull) ? 0x7FFFFFFF : 0; };
#pragma unroll 1
  for (int i0 = 0; i0 < kTileTokens; i0 += TB) {
    if (((vw >> (i0 + 1)) & ((1ull << TB) - 1ull)) == 0) continue;
    uint32_t code[TB][M];
#pragma unroll
    for (int k = 0; k < TB; ++k) {
      const buf_t src = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(cache) + readlane64(cbase, i0 + k + 1), 0,
                                                          records(i0 + k), 0x00020000);
#pragma unroll
      for (int m = 0; m < M; ++m) code[k][m] = __builtin_amdgcn_raw_buffer_load_b8(src, off(m, BS), 0, 0);
    }
#pragma unroll
    for (int k = 0; k < TB; ++k) {
      const buf_t dst = __builtin_amdgcn_make_buffer_rsrc(lin0 + static_cast<int64_t>(i0 + k) * a.lin_token_stride, 0,
                                                          records(i0 + k), 0x00020000);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const LutT v = lut_all[lut_off[m] + code[k][m]];
        if constexpr (ELT_L == 2) __builtin_amdgcn_raw_buffer_store_b16(v, dst, off(m, ELT_L), 0, kBufNT);
        else __builtin_amdgcn_raw_buffer_store_b32(v, dst, off(m, ELT_L), 0, kBufNT);
      }
    }
  }
}

// Launches of at most this many tokens take the TOKG instantiation; there a
// tile takes dequant_token_rows when its runs average fewer than
// kShortDequantRunTokens tokens and none goes on past the tile.
constexpr int64_t kTokenDequantTokens = 256;
constexpr int kShortDequantRunTokens = 3;

template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS, int STP, bool TOKG = false>
__global__ __launch_bounds__(kBlockThreads) void paged_wave_gather_kernel(const TileArgs a) {
  using W = WaveShape<ELT_C, ELT_L, BS>;
  constexpr int RPL = W::RPL, CG = W::CG, NCG = W::NCG, kChunkRows = W::kChunkRows;
  static_assert(kTileTokens + BS + 1 <= kWave, "run window must fit one wave");
  using LutT = typename LutEntry<ELT_L>::T;
  constexpr bool kLut = CODEC != kCopy;
  // Full runs stage the chunk through LDS (copies) or load lane tiles
  // directly (FP8, whose LDS holds the decode tables).
  constexpr bool kStage = !kLut;
  __shared__ u32x4 lds_all[kStage ? kWavesPerBlock * kWave * RPL : 1];
  __shared__ LutT lut_all[kLut ? kLutHeads * 256 : 1];
  u32x4* const lds = lds_all + wave_in_block() * (kWave * RPL);

  const int lane = lane_id();
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
  const int64_t t0 = tile * kTileTokens;
  const int plane = static_cast<int>(blockIdx.y);
  const int layer = plane >> 1;
  const int kv = plane & 1;
  const int64_t r0 = static_cast<int64_t>(blockIdx.z) * kChunkRows;  // this wave's cache rows
  const int64_t r_end = (r0 + kChunkRows < a.nrows) ? r0 + kChunkRows : a.nrows;

  // Slot window: lane i holds token t0 - 1 + i, and the runs of the tile.
  const int64_t t = t0 - 1 + lane;
  int64_t s = -1;
  if (t >= 0 && t < a.num_tokens) s = slot_at(a, t);
  const bool valid = (s >= 0) && (s < a.num_slots);
  const uint64_t vmask = ballot(valid);
  const int64_t s_prev = from_prev_lane(s);
  const bool prev_valid = lane > 0 && ((vmask >> (lane - 1)) & 1ull);
  const bool cont = valid && prev_valid && (s == s_prev + 1) && ((s % BS) != 0);
  const uint64_t cmask = ballot(cont);
  const int64_t remaining = a.num_tokens - t0;
  const int ntile = remaining <= 0 ? 0 : (remaining < kTileTokens ? static_cast<int>(remaining) : kTileTokens);
  const uint64_t window = ((1ull << ntile) - 1ull) << 1;
  uint64_t heads = vmask & ~cmask & window;

  uint8_t* const cache = a.cache[kv] + static_cast<int64_t>(layer) * a.cache_layer_stride;
  uint8_t* const lin = a.lin[kv] + static_cast<int64_t>(layer) * a.lin_layer_stride;
  const int rg = lane / NCG;  // lane tile: rows r0 + rg*RPL .., column group ct
  const int ct = lane % NCG;
  const int64_t trow = r0 + rg * RPL;
  const bool tile_in = trow < r_end;
  const uint32_t toff = static_cast<uint32_t>((rg * RPL * NCG + ct) * 16);

  // One run starting at lane i of the window: its block, columns and first token.
  struct Run {
    int64_t blk, tf;
    int c0, c1;
  };
  auto run_at = [&](int i) {
    const int len = 1 + __builtin_ctzll(~(cmask >> (i + 1)));  // i <= kTileTokens < 63
    const int64_t sh = readlane64(s, i);
    const int64_t blk = sh / BS;
    const int c0 = static_cast<int>(sh - blk * BS);
    return Run{blk, t0 - 1 + i, c0, c0 + len};
  };
  auto whole_chunk = [&](const Run& r) { return r.c0 < CG && r.c1 > BS - CG; };
  // FP8: each lane loads its own tile, RPL pieces 16 * NCG bytes apart.  A wave
  // instruction touches 64 lines partially; the loads are cached so that the L2
  // serves the rest of each line to the wave's next instructions.
  auto load_tile = [&](const Run& r, u32x4 (&d)[RPL]) {
    const buf_t cb = make_buf(cache + (r.blk * a.nrows + r0) * BS * ELT_C);
#pragma unroll
    for (int q = 0; q < RPL; ++q)
      d[q] = buf_ld16_cached(cb, tile_in ? toff + static_cast<uint32_t>(q * NCG * 16) : kOffOob);
  };

  // FP8: the first run's tile is loaded before the workgroup builds its decode
  // tables, so that the table work overlaps the loads' latency.
  u32x4 d[RPL];
  bool have_pre = false;
  if constexpr (kLut) {
    if (heads != 0) {
      const Run r = run_at(__builtin_ctzll(heads));
      if (whole_chunk(r)) {
        load_tile(r, d);
        have_pre = true;
      }
    }
  }

  // The workgroup's decode tables: its waves share the chunk (grid z), so the
  // heads h_lo .. of rows [r0, r_end) (one table for a scalar scale).  The
  // launcher routes chunks spanning more than kLutHeads heads elsewhere.
  const int h_lo = (kLut && a.scale_mode != 0) ? head_of_row(a, static_cast<int>(r0)) : 0;
  if constexpr (kLut) {
    const int nh = a.scale_mode != 0 ? head_of_row(a, static_cast<int>(r_end - 1)) - h_lo + 1 : 1;
    // Thread x writes code x of each table.  The heads' scales (load_scale's
    // indexing; indices past the last head repeat it, so every load stays in
    // the scale array) are all loaded before the first entry: the empty asm
    // statements keep the compiler from sinking each load, and its wait, into
    // its table's branch.
    static_assert(kBlockThreads == 256, "one code per thread and table");
    const float* const sp = a.scale[kv] + (a.scale_mode == 0   ? 0
                                           : a.scale_mode == 1 ? h_lo
                                                               : static_cast<int64_t>(layer) * a.num_heads + h_lo);
    float scs[kLutHeads];
#pragma unroll
    for (int k = 0; k < kLutHeads; ++k) scs[k] = sp[k < nh ? k : nh - 1];
#pragma unroll
    for (int k = 0; k < kLutHeads; ++k) asm volatile("" : "+v"(scs[k]));
#pragma unroll
    for (int k = 0; k < kLutHeads; ++k)
      if (k < nh) lut_all[k * 256 + threadIdx.x] = lut_value<CODEC, LDT, LutT>(threadIdx.x, scs[k]);
    __syncthreads();
  }
  if (t0 >= a.num_tokens) return;

  // The lane's table: all RPL rows of its tile lie in one head (head_dim is a
  // multiple of RPL on this path).
  const LutT* lut = lut_all;
  if (kLut && a.scale_mode != 0 && tile_in) lut += (head_of_row(a, static_cast<int>(trow)) - h_lo) * 256;

  if constexpr (TOKG && kLut) {
    // A whole tile of short runs (none going on past the tile) moves token by
    // token; the lanes of the runs that start in the tile are those a head's
    // next bit carries through in cmask.
    const uint64_t owned = heads | (((cmask + (heads << 1)) ^ cmask) & cmask);
    const int nr = __builtin_popcountll(heads);
    if (nr > 0 && (owned & ~window) == 0 && __builtin_popcountll(owned) < nr * kShortDequantRunTokens) {
      constexpr int M = kChunkRows / kWave;
      static_assert(kChunkRows % kWave == 0, "whole rows per lane");
      int lut_off[M];
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const int64_t row = r0 + m * kWave + lane;
        lut_off[m] = (a.scale_mode != 0 && row < r_end) ? (head_of_row(a, static_cast<int>(row)) - h_lo) * 256 : 0;
      }
      dequant_token_rows<ELT_L, BS, M, LutT>(a, cache, lin, lut_all, lut_off, s, owned, t0, r0, r_end);
      heads = 0;
    }
  }

  while (heads) {
    const int i = __builtin_ctzll(heads);
    heads &= heads - 1;
    const Run r = run_at(i);
    const int64_t blk = r.blk;
    const int c0 = r.c0;
    const int c1 = r.c1;
    const int64_t tf = r.tf;
    if (whole_chunk(r)) {
      // The run touches every column group: the whole chunk.  Loads and stores
      // go through wave-uniform buffer descriptors with per-lane 32-bit offsets
      // (kOffOob for masked lanes): no per-lane branches and no shared 64-bit
      // address registers, so the compiler issues all RPL loads back to back
      // and never waits on one access before the next address.
      if constexpr (kStage) {
        const buf_t cb = make_buf(cache + (blk * a.nrows + r0) * BS * ELT_C);
        u32x4 v[RPL];
#pragma unroll
        for (int k = 0; k < RPL; ++k) {
          const int pc = k * kWave + lane;
          v[k] = buf_ld16(cb, r0 + pc / NCG < r_end ? static_cast<uint32_t>(pc) * 16u : kOffOob);
        }
#pragma unroll
        for (int k = 0; k < RPL; ++k) lds[lds_slot<RPL, NCG>(k * kWave + lane)] = v[k];
        wave_lds_sync();
#pragma unroll
        for (int q = 0; q < RPL; ++q) d[q] = lds[lds_slot<RPL, NCG>((rg * RPL + q) * NCG + ct)];
        wave_lds_sync();
      } else {
        if (!have_pre) load_tile(r, d);  // the first run's tile is already loaded
        have_pre = false;
      }
      // The run's first token row at row r0; the lane's rows start rg * RPL
      // further.  Token offsets stay below 2 GiB (token stride <= 32 MiB).
      const buf_t lb = make_buf(lin + tf * a.lin_token_stride + r0 * ELT_L);
      const uint32_t lane_off = static_cast<uint32_t>(rg * RPL * ELT_L);
      const uint32_t stride32 = static_cast<uint32_t>(a.lin_token_stride);
#pragma unroll
      for (int cc = 0; cc < CG; ++cc) {
        const int c = ct * CG + cc;
        const bool mine = tile_in && c >= c0 && c < c1;
        buf_st16_p<STP>(lb, mine ? lane_off + static_cast<uint32_t>(c - c0) * stride32 : kOffOob,
                 gather_column<ELT_C, ELT_L, CODEC, RPL>(d, cc, lut));
      }
      continue;
    }

    // Short run: lane tiles over the rows of the chunk, one column group at a time.
    const int j0 = c0 / CG;
    const int j1 = (c1 - 1) / CG;
    for (int g = static_cast<int>(r0 / RPL) + lane; g < static_cast<int>(r_end / RPL); g += kWave) {
      const int64_t gr = static_cast<int64_t>(g) * RPL;
      const LutT* glut = lut_all;
      if (kLut && a.scale_mode != 0) glut += (head_of_row(a, static_cast<int>(gr)) - h_lo) * 256;
      uint8_t* const crow = cache + (blk * a.nrows + gr) * BS * ELT_C;
      uint8_t* const grow = lin + tf * a.lin_token_stride + gr * ELT_L;
#pragma unroll 1
      for (int j = j0; j <= j1; ++j) {
        const int lo = j * CG;
        u32x4 d[RPL];
#pragma unroll
        for (int q = 0; q < RPL; ++q) d[q] = ld16_cached(crow + (q * BS + lo) * ELT_C);
#pragma unroll
        for (int cc = 0; cc < CG; ++cc) {
          const int c = lo + cc;
          if (c >= c0 && c < c1)
            st16(grow + static_cast<int64_t>(c - c0) * a.lin_token_stride,
                 gather_column<ELT_C, ELT_L, CODEC, RPL>(d, cc, glut));
        }
      }
    }
  }

  if (a.fill_zeros) {
    uint64_t skipped = ~vmask & window;
    const u32x4 zero = {0u, 0u, 0u, 0u};
    while (skipped) {
      const int i = __builtin_ctzll(skipped);
      skipped &= skipped - 1;
      uint8_t* const row = lin + (t0 - 1 + i) * a.lin_token_stride;
      for (int64_t k = r0 * ELT_L + static_cast<int64_t>(lane) * 16; k < r_end * ELT_L; k += kWave * 16)
        st16(row + k, zero);
    }
  }
}

// ----- per-wave FP8 quant-store (linear -> paged) ---------------------------------------
//
// The mirror image of the gather.  Two lanes share one 16-column group of a
// block's cache rows: a lane takes RPL cache rows (one head) x 8 block
// columns of a run.  It loads the 8 linear pieces (RPL elements of one token
// each; a wave load instruction covers two tokens' 512 contiguous bytes),
// computes every quotient, and packs row q of four consecutive tokens into
// one dword with the hardware converter, so its half of row q's 16-byte cache
// piece leaves the converter already transposed.  The half pieces meet in
// the wave's LDS region (the gather's swizzle) and leave as coalesced 16-byte
// wave stores; runs that do not fill a whole block take the same steps and
// store only the bytes of their columns from those pieces.  The exactness
// conditions of the fast quotient and of the converter are checked per lane
// on the loaded inputs and made wave uniform; a wave that fails them encodes
// its columns element by element.

template <int ELT_L, int BS>
struct ScatterShape {
  static constexpr int RPL = 16 / ELT_L;                     // cache rows per lane tile
  static constexpr int CG = 16;                              // block columns per 16-byte group
  static constexpr int NCG = BS / CG;                        // 16-byte groups per cache row
  static constexpr int COLS = CG / 2;                        // block columns per lane
  static constexpr int kChunkRows = (kWave / (2 * NCG)) * RPL;
  static constexpr int kPieces = kChunkRows * NCG;           // 16-byte cache pieces per chunk
  static constexpr int kWaveChunks = 1;                      // chunks per wave (grid z covers the rest)
  static_assert(BS % CG == 0, "block row must be a whole number of 16-byte groups");
  static_assert(kPieces % kWave == 0, "chunk pieces must spread evenly over the wave");
};

// When a full-run tile may use the fast quotient and the converter (with
// the flush of sub-normal quotients), judged on the raw input bits of the
// lane.  The fast quotient is RN(x / s) for s and |x| in [2^-60, 2^60].
// 16-bit inputs only need the upper bound: every nonzero fp16 value is at
// least 2^-24, and a bf16 value below 2^-60 with s in [2^-45, 2^15] has a
// quotient below 2^-15 (flushed for both formats, like the exact quotient)
// and above 2^-149 (so its sign survives as in the exact quotient).
template <int LDT>
struct TileBound {
  uint32_t hi32 = 0u, lo32 = 0xFFFFFFFFu;
  u16x2 hi16 = {0, 0};

  __device__ __forceinline__ void add(const u32x4& v) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if constexpr (LDT == kLinF32) {
        const uint32_t a = v[w] & 0x7FFFFFFFu;
        lo32 = min(lo32, a - 1u);
        hi32 = max(hi32, a);
      } else {
        hi16 = __builtin_elementwise_max(hi16, __builtin_bit_cast(u16x2, v[w] & 0x7FFF7FFFu));
      }
    }
  }
  __device__ __forceinline__ uint32_t hi() const {
    if constexpr (LDT == kLinF32) return hi32;
    else return hi16.x > hi16.y ? hi16.x : hi16.y;
  }
  __device__ __forceinline__ bool fast(float s) const {
    if constexpr (LDT == kLinF32) {
      return fast_scale_ok(s) && lo32 >= kFastLoBits - 1u && hi32 < kFastHiBits;
    } else if constexpr (LDT == kLinBF16) {
      return (__float_as_uint(s) - 0x29000000u) < (0x47000000u - 0x29000000u) && hi() < (kFastHiBits >> 16);
    } else {
      return fast_scale_ok(s) && hi() < 0x7C00u;
    }
  }
  __device__ __forceinline__ float max_abs() const {
    if constexpr (LDT == kLinF32) return __uint_as_float(hi32);
    else if constexpr (LDT == kLinBF16) return bf16_bits_to_f32(hi());
    else return f16_bits_to_f32(hi());
  }
};

template <int CODEC, int LDT>
__device__ __forceinline__ uint32_t quant_soft(float x, float sc, float r, bool fast) {
  return fast ? fp8_encode_fast<CODEC>(quot_fast<LDT != kLinF32>(x, sc, r)) : fp8_encode<CODEC>(div_rn(x, sc));
}

// One element, checked on its own (edge columns of partial runs).
template <int CODEC, int LDT>
__device__ __forceinline__ uint32_t quant_one(float x, float sc, float r, bool scale_ok) {
  const uint32_t ax = __float_as_uint(x) & 0x7FFFFFFFu;
  const bool fast = scale_ok && (ax == 0u || (ax >= kFastLoBits && ax < kFastHiBits));
  return quant_soft<CODEC, LDT>(x, sc, r, fast);
}

template <int ELT_L, int LDT, int RPL>
__device__ __forceinline__ float tile_elem(const u32x4& piece, int q) {
  if constexpr (ELT_L == 2) return lin_to_f32<LDT>(elem16(piece, q));
  else return __uint_as_float(piece[q]);
}

// Quant-store tiles of short runs (a decode step's one to a few new tokens
// per sequence): instead of walking the runs one by one (a load round trip,
// the LDS exchange and the stores per run), the wave moves its chunk's rows of
// every such token at once, one row per lane: row r0 + m * 64 + lane of the
// token, M = kChunkRows / 64 rows per token.  The token is wave-uniform, so
// its linear row and its block column are scalar buffer descriptors (no
// records for a token that does not move) and a wave instruction covers 64
// consecutive rows: 64 elements of the linear row, 64 bytes of the block
// column at a row stride.  Every element is encoded on its own, as the
// element path of the run form does.  Lane i + 1 of `s` holds the slot of
// token t0 + i; bit i + 1 of `vw` says that the token moves.
template <int CODEC, int LDT, int ELT_L, int BS, int M>
__device__ __forceinline__ void quant_token_rows(const TileArgs& a, uint8_t* cache, const uint8_t* lin, int kv,
                                                 int layer, int64_t s, uint64_t vw, int64_t t0, int r0, int r_end) {
  constexpr int TB = 16 / M < kTileTokens ? 16 / M : kTileTokens;  // tokens per batch: 16 elements in flight per lane
  static_assert(kTileTokens % TB == 0, "whole batches");
  // The lane id and slot pass through an opaque copy, so that nothing derived
  // from them is hoisted out of the caller's chunk loop (it would stay live
  // across the run form and cost it a wave per SIMD).
  int lane = lane_id();
  asm volatile("" : "+v"(lane));
  asm volatile("" : "+v"(s));
  float sc[M], rc[M];
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int row = r0 + m * kWave + lane;
    sc[m] = row < r_end ? load_scale(a, kv, layer, head_of_row(a, row)) : 1.0f;
    rc[m] = fast_scale_ok(sc[m]) ? 1.0f / sc[m] : 0.0f;
  }
  auto off = [&](int m, int bytes) -> uint32_t {
    return r0 + m * kWave + lane < r_end ? static_cast<uint32_t>((m * kWave + lane) * bytes) : kOffOob;
  };
  const int64_t blk = s / BS;
  const int64_t cbase = (blk * a.nrows + r0) * BS + (s - blk * BS);
  const uint8_t* const lin0 = lin + t0 * a.lin_token_stride + static_cast<int64_t>(r0) * ELT_L;
  auto records = [&](int i) -> int { return ((vw >> (i + 1)) & 1ull) ? 0x7FFFFFFF : 0; };
#pragma unroll 1
  for (int i0 = 0; i0 < kTileTokens; i0 += TB) {
    if (((vw >> (i0 + 1)) & ((1ull << TB) - 1ull)) == 0) continue;
    uint32_t v[TB][M];
#pragma unroll
    for (int k = 0; k < TB; ++k) {
      const buf_t src = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<uint8_t*>(lin0) + static_cast<int64_t>(i0 + k) * a.lin_token_stride, 0, records(i0 + k),
          0x00020000);
#pragma unroll
      for (int m = 0; m < M; ++m) {
        if constexpr (ELT_L == 2) v[k][m] = __builtin_amdgcn_raw_buffer_load_b16(src, off(m, ELT_L), 0, kBufNT);
        else v[k][m] = __builtin_amdgcn_raw_buffer_load_b32(src, off(m, ELT_L), 0, kBufNT);
      }
    }
    auto elem = [&](uint32_t bits) { return ELT_L == 2 ? lin_to_f32<LDT>(bits) : __uint_as_float(bits); };
    auto cdesc = [&](int k) {
      return __builtin_amdgcn_make_buffer_rsrc(cache + readlane64(cbase, i0 + k + 1), 0, records(i0 + k),
                                               0x00020000);
    };
    // The fast quotient's range (quant_one's test), for the whole batch at once.
    bool fast = true;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      fast = fast && fast_scale_ok(sc[m]);
#pragma unroll
      for (int k = 0; k < TB; ++k) {
        const uint32_t ax = __float_as_uint(elem(v[k][m])) & 0x7FFFFFFFu;
        fast = fast && (ax == 0u || (ax >= kFastLoBits && ax < kFastHiBits));
      }
    }
    if (ballot(!fast) == 0) {
#pragma unroll
      for (int k = 0; k < TB; ++k) {
        const buf_t dst = cdesc(k);
#pragma unroll
        for (int m = 0; m < M; ++m) {
          const uint32_t code = fp8_encode_fast<CODEC>(quot_fast<LDT != kLinF32>(elem(v[k][m]), sc[m], rc[m]));
          __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(code), dst, off(m, BS), 0, 0);
        }
      }
    } else {
      // Some element needs the exact quotient: one element at a time, read
      // again, so that this rare path keeps few registers live.
#pragma unroll 1
      for (int k = 0; k < TB; ++k) {
        const buf_t src = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<uint8_t*>(lin0) + static_cast<int64_t>(i0 + k) * a.lin_token_stride, 0, records(i0 + k),
            0x00020000);
        const buf_t dst = cdesc(k);
#pragma unroll 1
        for (int m = 0; m < M; ++m) {
          const uint32_t x = ELT_L == 2 ? __builtin_amdgcn_raw_buffer_load_b16(src, off(m, ELT_L), 0, kBufNT)
                                        : __builtin_amdgcn_raw_buffer_load_b32(src, off(m, ELT_L), 0, kBufNT);
          float scm = sc[0], rcm = rc[0];
#pragma unroll
          for (int j = 1; j < M; ++j) {
            scm = m == j ? sc[j] : scm;
            rcm = m == j ? rc[j] : rcm;
          }
          const uint32_t code = quant_one<CODEC, LDT>(elem(x), scm, rcm, fast_scale_ok(scm));
          __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(code), dst, off(m, BS), 0, 0);
        }
      }
    }
  }
}

// Quant-store runs of a tile that average fewer than this many tokens take
// quant_token_rows.  Measured on one E4M3 layer ([8192, 8, 128, 16] cache,
// bf16 rows, per-head scales), per call: runs of 1-4 tokens faster at 16 to
// 4,096 tokens (single tokens 34.6 -> 11.0 us at 16, 61.4 -> 39.0 us at
// 4,096; runs of 4 24.7 -> 22.8 us at 4,096), runs of 6 level with 6 and 7 %
// slower with 8.
constexpr int kQuantShortRunTokens = 6;

// BM (block-major): the workgroups visit cache blocks in block order instead
// of token tiles (workgroup x owns block x, its four waves four consecutive
// row chunks of it), reading each block's claim tags as the inverse map of the
// scatter (see paged_block_scatter_kernel): the cache is then written in
// address order, and a workgroup reads its block's linear rows and writes its
// cache bytes as one contiguous span each.
template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS, bool BM>
__global__ __launch_bounds__(kBlockThreads) void paged_wave_scatter_kernel(const TileArgs a) {
  static_assert(ELT_C == 1 && CODEC != kCopy, "the per-wave scatter quantises into one-byte caches");
  using W = ScatterShape<ELT_L, BS>;
  constexpr int RPL = W::RPL, CG = W::CG, NCG = W::NCG, COLS = W::COLS;
  constexpr int kChunkRows = W::kChunkRows, kPieces = W::kPieces;
  static_assert(kTileTokens + BS + 1 <= kWave, "run window must fit one wave");
  __shared__ u32x4 lds_all[kWavesPerBlock * kPieces];
  u32x4* const lds = lds_all + wave_in_block() * kPieces;

  const int lane = lane_id();
  // Token order: wave w of workgroup x owns tile 4x + w, grid z its chunk.
  // Block order: workgroup x owns block x, its waves consecutive chunks.
  const int64_t unit = BM ? static_cast<int64_t>(blockIdx.x)
                          : static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
  const int chunk = BM ? static_cast<int>(blockIdx.z) * kWavesPerBlock + wave_in_block() : static_cast<int>(blockIdx.z);
  const int plane = static_cast<int>(blockIdx.y);
  const int layer = plane >> 1;
  const int kv = plane & 1;
  uint8_t* const cache = a.cache[kv] + static_cast<int64_t>(layer) * a.cache_layer_stride;
  const uint8_t* const lin = a.lin[kv] + static_cast<int64_t>(layer) * a.lin_layer_stride;
  // This wave's cache rows: up to W::kWaveChunks chunks of kChunkRows rows.
  const int rw0 = chunk * (kChunkRows * W::kWaveChunks);
  if (rw0 >= a.nrows) return;
  const int rw_end = (rw0 + kChunkRows * W::kWaveChunks < a.nrows) ? rw0 + kChunkRows * W::kWaveChunks
                                                                    : static_cast<int>(a.nrows);

  // Lane tile: rows trow .. trow + RPL - 1 of the chunk, block columns lo .. lo + COLS - 1
  // (rg here for the scales; each run derives the tile again).
  const int rg = (lane >> 1) / NCG;
  // The scale of the lane's rows in a chunk (1 for lanes past its end).  The
  // first chunk's is loaded before the slots or tags, so that the two loads
  // overlap instead of adding their latencies ahead of the linear loads.
  auto chunk_scale = [&](int r0) {
    const int r_end = (r0 + kChunkRows < rw_end) ? r0 + kChunkRows : rw_end;
    const int trow = r0 + rg * RPL;
    return trow < r_end ? load_scale(a, kv, layer, head_of_row(a, trow)) : 1.0f;
  };
  const float sc_first = chunk_scale(rw0);

  // Runs: `heads` marks the first lane of each, `cmask` the lanes continuing
  // one.
  uint64_t heads, cmask;
  uint64_t tok_lanes = 0;  // token order: lanes whose tokens take quant_token_rows
  int64_t s = -1, tok = -1;
  const int64_t t0 = unit * kTileTokens;
  if constexpr (!BM) {
    // Slot window: lane i holds token t0 - 1 + i; a token whose claim lost to a
    // later duplicate writes nothing.  The duplicate table is built by every
    // wave of the workgroup, before any of them leaves.
    if (a.scan_dupes) scan_build<kBlockThreads>(scan_table(), a);
    if (t0 >= a.num_tokens) return;
    const int64_t t = t0 - 1 + lane;
    if (t >= 0 && t < a.num_tokens) s = slot_at(a, t);
    bool valid = (s >= 0) && (s < a.num_slots);
    if (a.scan_dupes) {
      if (valid) valid = scan_is_last(scan_table(), s, t);
    } else if (valid && a.owner != nullptr) {
      valid = (a.owner[s] == claim_tag(a.epoch, t));
    }
    const uint64_t vmask = ballot(valid);
    const int64_t s_prev = from_prev_lane(s);
    const bool prev_valid = lane > 0 && ((vmask >> (lane - 1)) & 1ull);
    cmask = ballot(valid && prev_valid && (s == s_prev + 1) && ((s % BS) != 0));
    const int64_t remaining = a.num_tokens - t0;
    const int ntile = remaining < kTileTokens ? static_cast<int>(remaining) : kTileTokens;
    const uint64_t window = ((1ull << ntile) - 1ull) << 1;
    heads = vmask & ~cmask & window;
    // Lanes of the runs that start in this tile: adding a head's next bit to
    // cmask carries through exactly the continuation bits of its run.  A last
    // run that goes on past the tile's end keeps the run form; short runs
    // before it move with quant_token_rows.
    uint64_t tok_heads = heads;
    tok_lanes = heads | (((cmask + (heads << 1)) ^ cmask) & cmask);
    if (tok_lanes & ~window) {
      const uint64_t below_last = (1ull << (63 - __builtin_clzll(heads))) - 1ull;
      tok_heads &= below_last;
      tok_lanes &= below_last;
    }
    const int truns = __builtin_popcountll(tok_heads);
    if (truns > 0 && __builtin_popcountll(tok_lanes) < truns * kQuantShortRunTokens) heads &= ~tok_heads;
    else tok_lanes = 0;
  } else {
    // Lane p < BS holds the tag of slot unit * BS + p.
    if (unit * BS >= a.num_slots) return;
    uint64_t tag = 0;
    if (lane < BS) tag = a.owner[unit * BS + lane];
    const bool valid = lane < BS && static_cast<uint32_t>(tag >> 32) == a.epoch && static_cast<uint32_t>(tag) != 0u;
    tok = static_cast<int64_t>(static_cast<uint32_t>(tag)) - 1;
    const uint64_t vmask = ballot(valid);
    const int64_t tok_prev = from_prev_lane(tok);
    const bool prev_valid = lane > 0 && ((vmask >> (lane - 1)) & 1ull);
    cmask = ballot(valid && prev_valid && tok == tok_prev + 1);
    heads = vmask & ~cmask;
  }
  if (heads == 0 && tok_lanes == 0) return;

#pragma unroll 1
  for (int r0 = rw0; r0 < rw_end; r0 += kChunkRows) {
    const int r_end = (r0 + kChunkRows < rw_end) ? r0 + kChunkRows : rw_end;
    if constexpr (!BM) {
      static_assert(kChunkRows % kWave == 0, "whole rows per lane");
      if (tok_lanes != 0)
        quant_token_rows<CODEC, LDT, ELT_L, BS, kChunkRows / kWave>(a, cache, lin, kv, layer, s, tok_lanes, t0, r0,
                                                                    r_end);
    }
    const float sc = r0 == rw0 ? sc_first : chunk_scale(r0);
    const bool scale_ok = fast_scale_ok(sc);
    const float r = scale_ok ? 1.0f / sc : 0.0f;

    // One run: block columns [c0, c1) of block blk from tokens tf, tf + 1, ...
    auto run = [&](int64_t blk, int c0, int c1, int64_t tf) {
      // The lane's tile coordinates, derived again in every run from a lane id
      // the compiler cannot see through: hoisted out of the run loop, the
      // addresses built from them would stay live across every path and cost
      // a wave per SIMD.
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int half = ln & 1;
      const int rg = (ln >> 1) / NCG;
      const int ct = (ln >> 1) % NCG;
      const int lo = ct * CG + half * COLS;
      const int trow = r0 + rg * RPL;
      const bool tile_in = trow < r_end;
      u32x2* const lds_half = reinterpret_cast<u32x2*>(lds) + half;
      uint8_t* const chunk = cache + (blk * a.nrows + r0) * BS;
      const bool whole = c0 == 0 && c1 == BS;
      // Linear pieces: a descriptor at the run's first token and row r0 and a
      // per-lane offset (row group, column); lanes past the chunk, and columns
      // outside a partial run, read zeros.  All of a lane's pieces are loaded
      // at once, so a partial run costs one load latency like a whole block.
      const buf_t lbuf = make_buf(lin + tf * a.lin_token_stride + static_cast<int64_t>(r0) * ELT_L);
      const uint32_t stride32 = static_cast<uint32_t>(a.lin_token_stride);
      const uint32_t prow = static_cast<uint32_t>(rg * RPL * ELT_L);
      u32x4 in[COLS];
#pragma unroll
      for (int j = 0; j < COLS; ++j) {
        const int c = lo + j;
        const bool mine = tile_in && c >= c0 && c < c1;
        in[j] = buf_ld16(lbuf, mine ? prow + static_cast<uint32_t>(c - c0) * stride32 : kOffOob);
      }
      TileBound<LDT> bound;
#pragma unroll
      for (int c = 0; c < COLS; ++c) bound.add(in[c]);
      bool soft = !bound.fast(sc);
      if constexpr (CODEC == kE5M2) {
        // The converter is exact up to 57344; |q| <= max|x| * r * (1 + 2^-22).
        soft = soft || bound.max_abs() * r * (1.0f + 0x1p-20f) > __uint_as_float(kHwEncodeMaxBits<CODEC>);
      }
      // Row q of the lane's tile as two dwords of four block columns each.
      auto row_words = [&](int q, uint32_t (&word)[2]) {
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          float w[4];
#pragma unroll
          for (int k = 0; k < 4; ++k)
            w[k] = quot_fast<LDT != kLinF32>(tile_elem<ELT_L, LDT, RPL>(in[4 * g + k], q), sc, r);
          word[g] = fp8_pack4_hw<CODEC>(w[0], w[1], w[2], w[3]);
        }
      };
      if (ballot(tile_in && soft) == 0) {
        // The lanes' half pieces meet in LDS; whole blocks leave as coalesced
        // 16-byte stores, partial runs as the bytes of the run's columns of
        // the same coalesced pieces.
#pragma unroll
        for (int q = 0; q < RPL; ++q) {
          uint32_t word[2];
          row_words(q, word);
          lds_half[2 * lds_slot<RPL, NCG>((rg * RPL + q) * NCG + ct)] = u32x2{word[0], word[1]};
        }
        wave_lds_sync();
        const buf_t cbuf = make_buf(chunk);
#pragma unroll
        for (int k = 0; k < kPieces / kWave; ++k) {
          const int pc = k * kWave + lane;
          const u32x4 v = lds[lds_slot<RPL, NCG>(pc)];
          const bool row_in = r0 + pc / NCG < r_end;
          if (whole) {
            buf_st16(cbuf, row_in ? static_cast<uint32_t>(pc) * 16u : kOffOob, v);
          } else if (row_in) {
            // The piece's bytes inside the run: [b0, b1) of its 16 columns.
            const int cg0 = (pc % NCG) * CG;
            const int b0 = c0 > cg0 ? c0 - cg0 : 0;
            const int b1 = c1 < cg0 + CG ? c1 - cg0 : CG;
            uint8_t* const p = chunk + static_cast<int64_t>(pc) * 16;
#pragma unroll 1
            for (int b = b0; b < b1; ++b) {
              const uint32_t d = (b >> 2) == 0 ? v[0] : (b >> 2) == 1 ? v[1] : (b >> 2) == 2 ? v[2] : v[3];
              p[b] = static_cast<uint8_t>(d >> (8 * (b & 3)));
            }
          }
        }
        wave_lds_sync();
        return;
      }

      // Some lane of the wave needs the integer encoders: the lane's columns
      // inside the run, element by element, from the pieces already loaded
      // (no second round of loads: such waves would otherwise set the tail).
      // Columns and rows one at a time, the column's piece picked by selects,
      // so that this rare path keeps few registers live.
      if (!tile_in) return;
      const int ja = c0 > lo ? c0 - lo : 0;
      const int jb = c1 < lo + COLS ? c1 - lo : COLS;
      uint8_t* const crow = chunk + static_cast<int64_t>(rg * RPL) * BS + lo;
#pragma unroll 1
      for (int j = ja; j < jb; ++j) {
        u32x4 piece = in[0];
#pragma unroll
        for (int k = 1; k < COLS; ++k) piece = (j == k) ? in[k] : piece;
#pragma unroll 1
        for (int q = 0; q < RPL; ++q)
          crow[q * BS + j] =
              static_cast<uint8_t>(quant_one<CODEC, LDT>(tile_elem<ELT_L, LDT, RPL>(piece, q), sc, r, scale_ok));
      }
    };

    uint64_t hs = heads;
    while (hs) {
      const int i = __builtin_ctzll(hs);
      hs &= hs - 1;
      const int len = 1 + __builtin_ctzll(~(cmask >> (i + 1)));  // i < 63
      if constexpr (!BM) {
        const int64_t sh = readlane64(s, i);
        const int64_t blk = sh / BS;
        const int c0 = static_cast<int>(sh - blk * BS);
        run(blk, c0, c0 + len, t0 - 1 + i);
      } else {
        run(unit, i, i + len, readlane64(tok, i));
      }
    }
  }
}


// ----- per-wave 16-bit block-major scatter -----------------------------------------
//
// The bf16/fp16 scatter in destination order, shaped like the FP8 quant-store:
// workgroup x owns cache block x, its waves consecutive chunks of kChunkRows
// rows (grid z covers chunks past the fourth).  A lane loads 8 tokens' 16-byte
// linear pieces (8 rows each) of one run, transposes the 8 x 8 tile in
// registers into 8 cache pieces (8 tokens of one row each), and the pieces
// meet in the wave's LDS region to leave as coalesced 16-byte stores (whole
// blocks) or as the run's elements of those pieces (partial runs).  No
// workgroup barrier: each wave's LDS region is its own.
template <int BS>
struct CopyScatterShape {
  static constexpr int RPL = 8;                       // rows per linear piece (16-bit elements)
  static constexpr int CG = 8;                        // tokens per cache piece
  static constexpr int NCG = BS / CG;                 // cache pieces per cache row
  static constexpr int RG = kWave / NCG;              // lane row groups per wave
  static constexpr int kChunkRows = RG * RPL;         // cache rows per wave
  static constexpr int kPieces = kChunkRows * NCG;    // 16-byte cache pieces per wave
  static_assert(BS % CG == 0 && kWave % NCG == 0 && kPieces % kWave == 0, "block row of whole pieces");
};

template <int BS, int CSTP>
__global__ __launch_bounds__(kBlockThreads) void paged_wave_copy_scatter_kernel(const TileArgs a) {
  using W = CopyScatterShape<BS>;
  constexpr int ELT = 2, RPL = W::RPL, CG = W::CG, NCG = W::NCG, kChunkRows = W::kChunkRows;
  constexpr int kPieces = W::kPieces;
  __shared__ u32x4 lds_all[kWavesPerBlock * kPieces];
  u32x4* const lds = lds_all + wave_in_block() * kPieces;

  const int lane = lane_id();
  const int64_t blk = blockIdx.x;
  const int plane = static_cast<int>(blockIdx.y);
  const int layer = plane >> 1;
  const int kv = plane & 1;
  const int r0 = static_cast<int>(blockIdx.z) * (kWavesPerBlock * kChunkRows) + wave_in_block() * kChunkRows;
  if (r0 >= a.nrows || blk * BS >= a.num_slots) return;
  const int r_end = (r0 + kChunkRows < a.nrows) ? r0 + kChunkRows : static_cast<int>(a.nrows);

  // Lane p < BS holds the tag of slot blk * BS + p: runs of consecutive tokens.
  uint64_t tag = 0;
  if (lane < BS) tag = a.owner[blk * BS + lane];
  const bool valid = lane < BS && static_cast<uint32_t>(tag >> 32) == a.epoch && static_cast<uint32_t>(tag) != 0u;
  const int64_t tok = static_cast<int64_t>(static_cast<uint32_t>(tag)) - 1;
  const uint64_t vmask = ballot(valid);
  const int64_t tok_prev = from_prev_lane(tok);
  const bool prev_valid = lane > 0 && ((vmask >> (lane - 1)) & 1ull);
  const uint64_t cmask = ballot(valid && prev_valid && tok == tok_prev + 1);
  uint64_t heads = vmask & ~cmask;
  if (heads == 0) return;

  uint8_t* const cache = a.cache[kv] + static_cast<int64_t>(layer) * a.cache_layer_stride;
  const uint8_t* const lin = a.lin[kv] + static_cast<int64_t>(layer) * a.lin_layer_stride;
  uint8_t* const chunk = cache + (blk * a.nrows + r0) * (BS * ELT);
  const uint32_t stride32 = static_cast<uint32_t>(a.lin_token_stride);
  while (heads) {
    const int c0 = __builtin_ctzll(heads);
    heads &= heads - 1;
    const int c1 = c0 + 1 + __builtin_ctzll(~(cmask >> (c0 + 1)));  // c0 < BS <= 32
    const int64_t tf = readlane64(tok, c0);
    const bool whole = c0 == 0 && c1 == BS;
    // The lane's tile (rows rg*RPL .. of the chunk, tokens ct*CG ..), derived
    // in each run so that its addresses are not kept live across runs.
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int rg = ln / NCG;
    const int ct = ln % NCG;
    const bool tile_in = r0 + rg * RPL < r_end;
    const buf_t lbuf = make_buf(lin + tf * a.lin_token_stride + static_cast<int64_t>(r0) * ELT);
    const uint32_t prow = static_cast<uint32_t>(rg * RPL * ELT);
    u32x4 in[CG];
#pragma unroll
    for (int j = 0; j < CG; ++j) {
      const int c = ct * CG + j;
      const bool mine = tile_in && c >= c0 && c < c1;
      in[j] = buf_ld16(lbuf, mine ? prow + static_cast<uint32_t>(c - c0) * stride32 : kOffOob);
    }
#pragma unroll
    for (int q = 0; q < RPL; ++q) {
      u32x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = pack16(elem16(in[2 * k], q), elem16(in[2 * k + 1], q));
      lds[lds_slot<RPL, NCG>((rg * RPL + q) * NCG + ct)] = o;
    }
    wave_lds_sync();
    const buf_t cbuf = make_buf(chunk);
#pragma unroll
    for (int k = 0; k < kPieces / kWave; ++k) {
      const int pc = k * kWave + ln;
      const u32x4 v = lds[lds_slot<RPL, NCG>(pc)];
      const bool row_in = r0 + pc / NCG < r_end;
      if (whole) {
        buf_st16_p<CSTP>(cbuf, row_in ? static_cast<uint32_t>(pc) * 16u : kOffOob, v);
      } else if (row_in) {
        // The piece's elements inside the run: [e0, e1) of its 8 tokens.
        const int cg0 = (pc % NCG) * CG;
        const int e0 = c0 > cg0 ? c0 - cg0 : 0;
        const int e1 = c1 < cg0 + CG ? c1 - cg0 : CG;
#pragma unroll 1
        for (int e = e0; e < e1; ++e) {
          const uint32_t d = (e >> 1) == 0 ? v[0] : (e >> 1) == 1 ? v[1] : (e >> 1) == 2 ? v[2] : v[3];
          buf_st_elem<ELT>(cbuf, static_cast<uint32_t>(pc * 16 + e * ELT), half_of(d, e & 1));
        }
      }
    }
    wave_lds_sync();
  }
}
}  // namespace

// True when every linear token row covers whole 128-byte lines (row size,
// token and layer strides, both bases).
bool whole_line_rows(const TileArgs& a, int elt) {
  constexpr int64_t kLine = 128;
  return (a.nrows * elt) % kLine == 0 && a.lin_token_stride % kLine == 0 && a.lin_layer_stride % kLine == 0 &&
         reinterpret_cast<uintptr_t>(a.lin[0]) % kLine == 0 && reinterpret_cast<uintptr_t>(a.lin[1]) % kLine == 0;
}

// Dynamic LDS of the FP8 dequant-gather's workgroups, unused by the kernel:
// with its 4-8 KiB of decode tables, 3 workgroups fit in a CU's 160 KiB and 4
// do not.
constexpr unsigned kGatherLdsPad = 38000;
static_assert(4 * (kGatherLdsPad + kLutHeads * 256 * 2) > 160 * 1024 &&
                  3 * (kGatherLdsPad + kLutHeads * 256 * 4 + 16) <= 160 * 1024,
              "3 workgroups per CU, not 4");

template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS>
hipError_t launch_wave_gather(const TileArgs& a, int64_t planes, hipStream_t stream) {
  using W = WaveShape<ELT_C, ELT_L, BS>;
  const int64_t chunks = (a.nrows + W::kChunkRows - 1) / W::kChunkRows;
  if (chunks > 65535) return hipErrorInvalidValue;
  if (CODEC != kCopy && a.scale_mode != 0) {
    // Every chunk's heads must fit the workgroup's decode tables.
    for (int64_t z = 0; z < chunks; ++z) {
      const int64_t r0 = z * W::kChunkRows;
      const int64_t r1 = (r0 + W::kChunkRows < a.nrows ? r0 + W::kChunkRows : a.nrows) - 1;
      if (r1 / a.head_dim - r0 / a.head_dim + 1 > kLutHeads) return hipErrorNotSupported;
    }
  }
  const int64_t tiles = (a.num_tokens + kTileTokens - 1) / kTileTokens;
  const int64_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid(static_cast<uint32_t>(blocks), static_cast<uint32_t>(planes), static_cast<uint32_t>(chunks));
  // Linear rows of whole lines are written through the L2 (cfg 3
  // dequant-gather 5.39 -> 5.48 TB/s, caches read from HBM).  Each wave
  // instruction touches 64 cache lines partially and the wave's next ones
  // read the rest, so fewer waves per CU keep more of those lines in the L1:
  // the launch adds dynamic LDS (kGatherLdsPad, unused) so that 3 workgroups
  // fit per CU.  Measured on cfg 3 against 4 per CU (two runs): per-head
  // scales +0.8-1.3 % (E4M3) and +1.5 % (E5M2), scalar scale and the dense
  // FP8 preload -0.3-0.5 %;
  // 5 per CU was 2-5 % slower, and staging the tiles through LDS with
  // whole-line loads gained 1.6 % on cfg 3 but lost 6 % on the dense preload.
  const bool tok = a.num_tokens <= kTokenDequantTokens;
  if (whole_line_rows(a, ELT_L) && tok)
    hipLaunchKernelGGL((paged_wave_gather_kernel<ELT_C, ELT_L, CODEC, LDT, BS, kBufWT, true>), grid,
                       dim3(kBlockThreads), kGatherLdsPad, stream, a);
  else if (whole_line_rows(a, ELT_L))
    hipLaunchKernelGGL((paged_wave_gather_kernel<ELT_C, ELT_L, CODEC, LDT, BS, kBufWT>), grid, dim3(kBlockThreads),
                       kGatherLdsPad, stream, a);
  else if (tok)
    hipLaunchKernelGGL((paged_wave_gather_kernel<ELT_C, ELT_L, CODEC, LDT, BS, kBufNT, true>), grid,
                       dim3(kBlockThreads), kGatherLdsPad, stream, a);
  else
    hipLaunchKernelGGL((paged_wave_gather_kernel<ELT_C, ELT_L, CODEC, LDT, BS, kBufNT>), grid, dim3(kBlockThreads),
                       kGatherLdsPad, stream, a);
  return hipGetLastError();
}

template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS>
hipError_t launch_wave_scatter(const TileArgs& a, int64_t planes, hipStream_t stream) {
  using W = ScatterShape<ELT_L, BS>;
  const int64_t chunks = (a.nrows + W::kChunkRows * W::kWaveChunks - 1) / (W::kChunkRows * W::kWaveChunks);
  if (chunks > 65535) return hipErrorInvalidValue;
  // Block order when the claim tags are this call's inverse map and the tokens
  // cover a good share of the slots (as for the 16- and 32-bit scatter).
  const bool bm = a.owner != nullptr && a.owner_exclusive && a.num_tokens * 4 >= a.num_slots;
  const int64_t blocks = bm ? a.num_slots / BS : ((a.num_tokens + kTileTokens - 1) / kTileTokens + kWavesPerBlock - 1) /
                                                     kWavesPerBlock;
  const int64_t zs = bm ? (chunks + kWavesPerBlock - 1) / kWavesPerBlock : chunks;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid(static_cast<uint32_t>(blocks), static_cast<uint32_t>(planes), static_cast<uint32_t>(zs));
  // In block order one workgroup takes one block (grid z covers chunks past
  // the fourth) and the lane's scale load is issued before the tag load: on
  // configs[2]'s quant-store 5.04-5.16 -> 5.21-5.38 TB/s, where either change
  // alone measured no faster.  Partial runs (a sequence's last block) once
  // loaded and encoded their columns one load at a time: those few waves ran
  // several load latencies long and set the kernel's tail; sharing the
  // whole-block path moved the quant-store on to 5.42-5.75 TB/s.  Slower in
  // the same runs: two or four blocks per wave under one tag load (-2 % /
  // -7 %), four lanes per 16-byte group (69 VGPRs, 7 waves per SIMD; -2 %),
  // one lane per group (whole 1 KiB loads, 142 VGPRs, 3 waves per SIMD;
  // -6 %), at most 4 or 3 workgroups per CU (-2 % / -9 %), cached or sc0
  // linear loads (-4 %), write-back cache stores (-8 %); 6 waves per SIMD (79
  // VGPRs: row groups padded in LDS so that the lanes' LDS and store addresses
  // take immediate offsets) and write-through stores were level.
  if (bm)
    hipLaunchKernelGGL((paged_wave_scatter_kernel<ELT_C, ELT_L, CODEC, LDT, BS, true>), grid, dim3(kBlockThreads), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((paged_wave_scatter_kernel<ELT_C, ELT_L, CODEC, LDT, BS, false>), grid, dim3(kBlockThreads), 0,
                       stream, a);
  return hipGetLastError();
}

template <int BS>
hipError_t launch_wave_copy_scatter(const TileArgs& a, int64_t planes, hipStream_t stream) {
  using W = CopyScatterShape<BS>;
  const int64_t chunks = (a.nrows + W::kChunkRows - 1) / W::kChunkRows;
  const int64_t zs = (chunks + kWavesPerBlock - 1) / kWavesPerBlock;
  const int64_t nblk = a.num_slots / BS;
  if (zs > 65535 || nblk > 0x7FFFFFFF) return hipErrorInvalidValue;
  // Whole blocks are written through the L2, as in the cooperative kernel.
  const dim3 grid(static_cast<uint32_t>(nblk), static_cast<uint32_t>(planes), static_cast<uint32_t>(zs));
  hipLaunchKernelGGL((paged_wave_copy_scatter_kernel<BS, kBufWT>), grid, dim3(kBlockThreads), 0, stream, a);
  return hipGetLastError();
}
template hipError_t launch_wave_copy_scatter<8>(const TileArgs&, int64_t, hipStream_t);
template hipError_t launch_wave_copy_scatter<16>(const TileArgs&, int64_t, hipStream_t);
template hipError_t launch_wave_copy_scatter<32>(const TileArgs&, int64_t, hipStream_t);

#define KVHIP_WAVE_GATHER(CODEC, ELT_L, LDT)                                                             \
  template hipError_t launch_wave_gather<1, ELT_L, CODEC, LDT, 16>(const TileArgs&, int64_t, hipStream_t);  \
  template hipError_t launch_wave_gather<1, ELT_L, CODEC, LDT, 32>(const TileArgs&, int64_t, hipStream_t);  \
  template hipError_t launch_wave_scatter<1, ELT_L, CODEC, LDT, 16>(const TileArgs&, int64_t, hipStream_t); \
  template hipError_t launch_wave_scatter<1, ELT_L, CODEC, LDT, 32>(const TileArgs&, int64_t, hipStream_t);
KVHIP_WAVE_GATHER(kE4M3, 2, kLinBF16)
KVHIP_WAVE_GATHER(kE4M3, 2, kLinF16)
KVHIP_WAVE_GATHER(kE4M3, 4, kLinF32)
KVHIP_WAVE_GATHER(kE5M2, 2, kLinBF16)
KVHIP_WAVE_GATHER(kE5M2, 2, kLinF16)
KVHIP_WAVE_GATHER(kE5M2, 4, kLinF32)
#undef KVHIP_WAVE_GATHER

}  // namespace kvhip
