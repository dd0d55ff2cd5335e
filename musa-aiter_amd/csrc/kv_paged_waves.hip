// Per-wave paged-A -> linear gather for MI355X (gfx950), used for the FP8
// dequant-gather.
//
// One wave owns the runs (consecutive tokens in consecutive slots of one
// block) that start in its 16-token tile, for one chunk of cache rows (grid z).
// A chunk is 64 lane tiles of RPL rows x CG block columns, i.e. RPL KiB of
// contiguous cache bytes: the cache side moves as RPL coalesced wave loads
// (lane l takes piece k*64 + l), the pieces are exchanged through the wave's
// private LDS region so that each lane holds an RPL x CG tile, and the lane
// transposes its tile in registers while decoding (byte selects, decode,
// scale, round), writing 16-byte pieces of token rows.  For one-byte cache
// elements this needs RPL / (RPL * CG) = 1/16 LDS instruction per element,
// against the 1 to 1.25 of the workgroup-cooperative kernel's column reads,
// which makes it the faster dequant-gather.  Runs that do not cover every
// column group of the block row use lane tiles directly and load only the
// column groups they cover.
#include "kv_hip_common.h"
#include "kv_launch.h"
#include "kv_paged_args.h"

namespace kvhip {

namespace {

// d[q] holds 16 bytes of cache row (r0+q) for one column group; returns the
// 16-byte linear piece (rows r0..r0+RPL-1) of block column `cc`.
template <int ELT_C, int ELT_L, int CODEC, int LDT, int RPL>
__device__ __forceinline__ u32x4 gather_column(const u32x4 (&d)[RPL], int cc, float sc) {
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
      for (int k = 0; k < 4; ++k) {
        const uint32_t lo = f32_to_lin<LDT>(fp8_decode<CODEC>(elem8(d[2 * k], cc)) * sc);
        const uint32_t hi = f32_to_lin<LDT>(fp8_decode<CODEC>(elem8(d[2 * k + 1], cc)) * sc);
        o[k] = pack16(lo, hi);
      }
    } else {
#pragma unroll
      for (int k = 0; k < 4; ++k) o[k] = __float_as_uint(fp8_decode<CODEC>(elem8(d[k], cc)) * sc);
    }
  }
  return o;
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

template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS>
__global__ __launch_bounds__(kBlockThreads) void paged_wave_gather_kernel(const TileArgs a) {
  using W = WaveShape<ELT_C, ELT_L, BS>;
  constexpr int RPL = W::RPL, CG = W::CG, NCG = W::NCG, kChunkRows = W::kChunkRows;
  static_assert(kTileTokens + BS + 1 <= kWave, "run window must fit one wave");
  __shared__ u32x4 lds_all[kWavesPerBlock * kWave * RPL];
  u32x4* const lds = lds_all + wave_in_block() * (kWave * RPL);

  const int lane = lane_id();
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
  const int64_t t0 = tile * kTileTokens;
  if (t0 >= a.num_tokens) return;
  const int plane = static_cast<int>(blockIdx.y);
  const int layer = plane >> 1;
  const int kv = plane & 1;
  uint8_t* const cache = a.cache[kv] + static_cast<int64_t>(layer) * a.cache_layer_stride;
  uint8_t* const lin = a.lin[kv] + static_cast<int64_t>(layer) * a.lin_layer_stride;
  const int64_t r0 = static_cast<int64_t>(blockIdx.z) * kChunkRows;  // this wave's cache rows
  const int64_t r_end = (r0 + kChunkRows < a.nrows) ? r0 + kChunkRows : a.nrows;

  // Slot window: lane i holds token t0 - 1 + i.
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
  const int ntile = remaining < kTileTokens ? static_cast<int>(remaining) : kTileTokens;
  const uint64_t window = ((1ull << ntile) - 1ull) << 1;
  uint64_t heads = vmask & ~cmask & window;

  const int rg = lane / NCG;  // lane tile: rows r0 + rg*RPL .., column group ct
  const int ct = lane % NCG;
  const int64_t trow = r0 + rg * RPL;
  const bool tile_in = trow < r_end;
  float sc = 1.0f;
  if constexpr (CODEC != kCopy) {
    if (tile_in) sc = load_scale(a, kv, layer, trow / a.head_dim);
  }

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
    uint8_t* const chunk = cache + (blk * a.nrows + r0) * BS * ELT_C;
    uint8_t* const lrow = lin + tf * a.lin_token_stride + trow * ELT_L;

    if (c0 < CG && c1 > BS - CG) {
      // The run touches every column group: stage the whole chunk.
      u32x4 v[RPL];
#pragma unroll
      for (int k = 0; k < RPL; ++k) {
        const int pc = k * kWave + lane;
        if (r0 + pc / NCG < r_end) v[k] = ld16(chunk + pc * 16);
      }
#pragma unroll
      for (int k = 0; k < RPL; ++k) lds[lds_slot<RPL, NCG>(k * kWave + lane)] = v[k];
      wave_lds_sync();
      u32x4 d[RPL];
#pragma unroll
      for (int q = 0; q < RPL; ++q) d[q] = lds[lds_slot<RPL, NCG>((rg * RPL + q) * NCG + ct)];
      wave_lds_sync();
      if (tile_in) {
#pragma unroll
        for (int cc = 0; cc < CG; ++cc) {
          const int c = ct * CG + cc;
          if (c >= c0 && c < c1)
            st16(lrow + static_cast<int64_t>(c - c0) * a.lin_token_stride,
                 gather_column<ELT_C, ELT_L, CODEC, LDT, RPL>(d, cc, sc));
        }
      }
      continue;
    }

    // Short run: lane tiles over the rows of the chunk, one column group at a time.
    const int j0 = c0 / CG;
    const int j1 = (c1 - 1) / CG;
    for (int g = static_cast<int>(r0 / RPL) + lane; g < static_cast<int>(r_end / RPL); g += kWave) {
      const int64_t gr = static_cast<int64_t>(g) * RPL;
      float gsc = 1.0f;
      if constexpr (CODEC != kCopy) gsc = load_scale(a, kv, layer, gr / a.head_dim);
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
                 gather_column<ELT_C, ELT_L, CODEC, LDT, RPL>(d, cc, gsc));
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

}  // namespace

template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS>
hipError_t launch_wave_gather(const TileArgs& a, int64_t planes, hipStream_t stream) {
  using W = WaveShape<ELT_C, ELT_L, BS>;
  const int64_t chunks = (a.nrows + W::kChunkRows - 1) / W::kChunkRows;
  if (chunks > 65535) return hipErrorInvalidValue;
  const int64_t tiles = (a.num_tokens + kTileTokens - 1) / kTileTokens;
  const int64_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  hipLaunchKernelGGL((paged_wave_gather_kernel<ELT_C, ELT_L, CODEC, LDT, BS>),
                     dim3(static_cast<uint32_t>(blocks), static_cast<uint32_t>(planes), static_cast<uint32_t>(chunks)),
                     dim3(kBlockThreads), 0, stream, a);
  return hipGetLastError();
}

#define KVHIP_WAVE_GATHER(CODEC, ELT_L, LDT)                                                            \
  template hipError_t launch_wave_gather<1, ELT_L, CODEC, LDT, 16>(const TileArgs&, int64_t, hipStream_t); \
  template hipError_t launch_wave_gather<1, ELT_L, CODEC, LDT, 32>(const TileArgs&, int64_t, hipStream_t);
KVHIP_WAVE_GATHER(kE4M3, 2, kLinBF16)
KVHIP_WAVE_GATHER(kE4M3, 2, kLinF16)
KVHIP_WAVE_GATHER(kE4M3, 4, kLinF32)
KVHIP_WAVE_GATHER(kE5M2, 2, kLinBF16)
KVHIP_WAVE_GATHER(kE5M2, 2, kLinF16)
KVHIP_WAVE_GATHER(kE5M2, 4, kLinF32)
#undef KVHIP_WAVE_GATHER

}  // namespace kvhip
