// Paged-A KV cache <-> token-major linear transfers for MI355X (gfx950).
//
// Cache layout (the reference API layout, musa_aiter/ops/kv_transfer.py:3-14):
//   [NL, NB, NH, HD, BS]  -- block_size innermost, so one token's head row is
//   strided by BS elements.  Linear layout: [.., T, NH, HD] token-major rows.
//
// Design.  A "run" is a maximal set of consecutive tokens whose slots are
// consecutive inside one block (tokens of one sequence filling one block).
// One wave owns the runs that start inside its 16-token tile.  For a run the
// wave walks the NH*HD cache rows in lane tiles of RPL rows x (16 bytes of
// block columns): every lane issues RPL 16-byte loads of block rows, transposes
// the tile in registers (v_perm byte selects, no LDS), applies the fused FP8
// codec if any, and writes 16-byte pieces of token rows.  Both the loads and
// the stores are full 16-byte vectors; partial column groups only occur at the
// first/last block of a sequence, where the scatter falls back to element
// stores so neighbouring slots are never touched.
//
// Slots are resolved once per wave (one 64-lane window load), K and V and the
// layers are separate grid planes, and skipped tokens (slot < 0) are zero
// filled by the wave that owns them.
#include "kv_hip_common.h"
#include "kv_launch.h"

namespace kvhip {

struct TileArgs {
  uint8_t* cache[2];
  uint8_t* lin[2];
  const int64_t* slots;
  const float* scale[2];
  const uint64_t* owner;
  int64_t num_tokens;
  int64_t num_slots;
  int64_t nrows;               // NH * HD
  int64_t head_dim;
  int64_t num_heads;
  int64_t cache_layer_stride;  // bytes
  int64_t lin_layer_stride;    // bytes
  int64_t lin_token_stride;    // bytes
  int32_t scale_mode;
  int32_t fill_zeros;
  uint32_t epoch;
  int32_t block_size;          // used by the generic kernel only
  int64_t split_rows;          // cache rows per grid z-slice (tile kernel)
};

constexpr int kTileTokens = 16;

__device__ __forceinline__ float load_scale(const TileArgs& a, int kv, int layer, int64_t head) {
  const float* s = a.scale[kv];
  if (a.scale_mode == 0) return s[0];
  if (a.scale_mode == 1) return s[head];
  return s[static_cast<int64_t>(layer) * a.num_heads + head];
}

// ----- lane-tile transposes ---------------------------------------------------

// Gather: d[q] holds 16 bytes of cache row (r0+q) for one column group; return
// the 16-byte linear piece (rows r0..r0+RPL-1) of block column `cc`.
template <int ELT_C, int ELT_L, int CODEC, int LDT, int RPL>
__device__ __forceinline__ u32x4 gather_column(const u32x4 (&d)[RPL], int cc, float sc) {
  u32x4 o;
  if constexpr (CODEC == kCopy && ELT_C == 2) {
    static_assert(RPL == 8, "bf16/fp16 tiles are 8x8");
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

// Scatter: in[cc] holds the 16-byte linear piece (rows r0..r0+RPL-1) of the
// token in block column cc; element (q, cc) of the tile in cache encoding.
// FAST selects the hoisted-reciprocal quotient (r = RN(1/sc)); the caller
// guarantees the fast range for the scale and every input of the tile.
template <int ELT_C, int ELT_L, int CODEC, int LDT, bool FAST = false>
__device__ __forceinline__ uint32_t scatter_elem(const u32x4& in_cc, int q, float sc, float r = 0.0f) {
  if constexpr (CODEC == kCopy && ELT_C == 2) {
    return elem16(in_cc, q);
  } else if constexpr (CODEC == kCopy && ELT_C == 4) {
    return in_cc[q];
  } else {
    float x;
    if constexpr (ELT_L == 2) x = lin_to_f32<LDT>(elem16(in_cc, q));
    else x = __uint_as_float(in_cc[q]);
    if constexpr (FAST) return fp8_encode_fast<CODEC>(quot_fast(x, sc, r));
    else return fp8_encode<CODEC>(div_rn(x, sc));
  }
}

template <int ELT_C, int ELT_L, int CODEC, int LDT, int CG, bool FAST = false>
__device__ __forceinline__ u32x4 scatter_row(const u32x4 (&in)[CG], int q, float sc, float r = 0.0f) {
  u32x4 o;
  if constexpr (ELT_C == 2) {
#pragma unroll
    for (int w = 0; w < 4; ++w)
      o[w] = pack16(scatter_elem<ELT_C, ELT_L, CODEC, LDT, FAST>(in[2 * w], q, sc, r),
                    scatter_elem<ELT_C, ELT_L, CODEC, LDT, FAST>(in[2 * w + 1], q, sc, r));
  } else if constexpr (ELT_C == 4) {
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = scatter_elem<ELT_C, ELT_L, CODEC, LDT, FAST>(in[w], q, sc, r);
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      uint32_t acc = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b)
        acc |= scatter_elem<ELT_C, ELT_L, CODEC, LDT, FAST>(in[4 * w + b], q, sc, r) << (8 * b);
      o[w] = acc;
    }
  }
  return o;
}

// Writes the RPL cache rows of one lane tile through `put(q, row)`.  FP8
// tiles whose scale and inputs are all in the fast range use the hoisted
// reciprocal; any other tile divides exactly.
template <int ELT_C, int ELT_L, int CODEC, int LDT, int CG, int RPL, typename Put>
__device__ __forceinline__ void encode_tile(const u32x4 (&in)[CG], float sc, Put put) {
  if constexpr (CODEC == kCopy) {
#pragma unroll
    for (int q = 0; q < RPL; ++q) put(q, scatter_row<ELT_C, ELT_L, CODEC, LDT, CG>(in, q, sc));
  } else {
    InputRange<LDT> range;
#pragma unroll
    for (int cc = 0; cc < CG; ++cc) range.add(in[cc]);
    if (fast_scale_ok(sc) && range.in_fast_range()) {
      const float r = 1.0f / sc;
#pragma unroll
      for (int q = 0; q < RPL; ++q) put(q, scatter_row<ELT_C, ELT_L, CODEC, LDT, CG, true>(in, q, sc, r));
    } else {
#pragma unroll
      for (int q = 0; q < RPL; ++q) put(q, scatter_row<ELT_C, ELT_L, CODEC, LDT, CG>(in, q, sc));
    }
  }
}

template <int ELT>
__device__ __forceinline__ void store_elem(uint8_t* p, uint32_t v) {
  if constexpr (ELT == 1) *p = static_cast<uint8_t>(v);
  else if constexpr (ELT == 2) *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(v);
  else *reinterpret_cast<uint32_t*>(p) = v;
}

// Element `idx` of a 16-byte cache piece, in cache encoding.
template <int ELT>
__device__ __forceinline__ uint32_t piece_elem(const u32x4& v, int idx) {
  if constexpr (ELT == 1) return elem8(v, idx);
  else if constexpr (ELT == 2) return elem16(v, idx);
  else return v[idx];
}

// ----- LDS staging of one block run ----------------------------------------------
//
// A chunk is 64 lane tiles of RPL rows x CG block columns: kChunkRows cache
// rows of one block, i.e. RPL KiB of contiguous cache bytes.  The cache side
// of a chunk moves as RPL coalesced wave instructions (lane l takes piece
// k*64 + l); the lane tiles are exchanged through the wave's private LDS
// region, so both the cache and the linear side issue whole cache lines.
// Piece s of the chunk lives at LDS slot lds_slot(s): the low four bits are
// XOR-swizzled with the row group so that 16 consecutive lanes hit 16
// distinct 16-byte bank groups in both access patterns.

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

template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS, bool SCATTER>
__device__ __forceinline__ void staged_run(const TileArgs& a, uint8_t* const cache_blk, uint8_t* const lin_run,
                                           const int c0, const int c1, const int kv, const int layer,
                                           u32x4* const lds, const int64_t r_begin, const int64_t r_end,
                                           const int rot) {
  constexpr int RPL = 16 / ELT_L;
  constexpr int CG = 16 / ELT_C;
  constexpr int NCG = BS / CG;
  constexpr int kChunkRows = (kWave / NCG) * RPL;
  const int lane = lane_id();
  const int rg = lane / NCG;
  const int ct = lane % NCG;
  const bool full = (c0 == 0) && (c1 == BS);

  // Chunks are visited starting at chunk `rot` (different per wave), so the
  // waves in flight spread over all address phases of the block and of the
  // token rows instead of all streaming the same offsets at the same time.
  const int nchunks = static_cast<int>((r_end - r_begin + kChunkRows - 1) / kChunkRows);
  int chunk_id = rot % nchunks;
  for (int ci = 0; ci < nchunks; ++ci, chunk_id = (chunk_id + 1 == nchunks) ? 0 : chunk_id + 1) {
    const int64_t r0 = r_begin + static_cast<int64_t>(chunk_id) * kChunkRows;
    uint8_t* const chunk = cache_blk + r0 * BS * ELT_C;
    const int64_t trow = r0 + rg * RPL;  // first cache row of this lane's tile
    const bool tile_in = trow < a.nrows;
    float sc = 1.0f;
    if constexpr (CODEC != kCopy) {
      if (tile_in) sc = load_scale(a, kv, layer, trow / a.head_dim);
    }
    uint8_t* const lrow = lin_run + trow * ELT_L;

    if constexpr (!SCATTER) {
      u32x4 v[RPL];
#pragma unroll
      for (int k = 0; k < RPL; ++k) {
        const int pc = k * kWave + lane;
        if (r0 + pc / NCG < a.nrows) v[k] = ld16(chunk + pc * 16);
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
    } else {
      u32x4 in[CG];
#pragma unroll
      for (int cc = 0; cc < CG; ++cc) {
        const int c = ct * CG + cc;
        in[cc] = u32x4{0u, 0u, 0u, 0u};
        if (tile_in && c >= c0 && c < c1) in[cc] = ld16(lrow + static_cast<int64_t>(c - c0) * a.lin_token_stride);
      }
      encode_tile<ELT_C, ELT_L, CODEC, LDT, CG, RPL>(
          in, sc, [&](int q, const u32x4& row) { lds[lds_slot<RPL, NCG>((rg * RPL + q) * NCG + ct)] = row; });
      wave_lds_sync();
#pragma unroll
      for (int k = 0; k < RPL; ++k) {
        const int pc = k * kWave + lane;
        const u32x4 w = lds[lds_slot<RPL, NCG>(pc)];
        if (r0 + pc / NCG >= a.nrows) continue;
        uint8_t* const dst = chunk + pc * 16;
        const int lo = (pc % NCG) * CG;
        if (full || (lo >= c0 && lo + CG <= c1)) {
          st16(dst, w);
        } else {
#pragma unroll
          for (int cc = 0; cc < CG; ++cc)
            if (lo + cc >= c0 && lo + cc < c1) store_elem<ELT_C>(dst + cc * ELT_C, piece_elem<ELT_C>(w, cc));
        }
      }
      wave_lds_sync();
    }
  }
}

// ----- the tile kernel ---------------------------------------------------------

template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS, bool SCATTER>
__global__ __launch_bounds__(kBlockThreads) void paged_tile_kernel(const TileArgs a) {
  constexpr int RPL = 16 / ELT_L;  // cache rows per lane tile
  constexpr int CG = 16 / ELT_C;   // block columns per 16-byte group
  static_assert(BS % CG == 0, "block row must be a whole number of 16-byte groups");
  static_assert(kTileTokens + BS + 1 <= kWave, "run window must fit one wave");

  const int lane = lane_id();
  const int64_t tile = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave_in_block();
  const int64_t t0 = tile * kTileTokens;
  if (t0 >= a.num_tokens) return;
  const int plane = static_cast<int>(blockIdx.y);
  const int layer = plane >> 1;
  const int kv = plane & 1;
  uint8_t* const cache = a.cache[kv] + static_cast<int64_t>(layer) * a.cache_layer_stride;
  uint8_t* const lin = a.lin[kv] + static_cast<int64_t>(layer) * a.lin_layer_stride;
  // The z-slice of the grid picks a range of cache rows (a whole number of
  // LDS chunks), so one run is spread over several independent waves.
  const int64_t r_begin = static_cast<int64_t>(blockIdx.z) * a.split_rows;
  const int64_t r_end = (r_begin + a.split_rows < a.nrows) ? r_begin + a.split_rows : a.nrows;

  // Slot window: lane i holds token t0 - 1 + i.
  const int64_t t = t0 - 1 + lane;
  int64_t s = -1;
  if (t >= 0 && t < a.num_tokens) s = a.slots[t];
  bool valid = (s >= 0) && (s < a.num_slots);
  if constexpr (SCATTER) {
    if (valid && a.owner != nullptr) valid = (a.owner[s] == claim_tag(a.epoch, t));
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

  const int ngroups = static_cast<int>(r_end / RPL);
  __shared__ u32x4 lds_all[kWavesPerBlock * kWave * RPL];
  u32x4* const lds = lds_all + wave_in_block() * (kWave * RPL);

  while (heads) {
    const int i = __builtin_ctzll(heads);
    heads &= heads - 1;
    const uint64_t after = cmask >> (i + 1);  // i <= kTileTokens < 63
    const int len = 1 + __builtin_ctzll(~after);
    const int64_t sh = readlane64(s, i);
    const int64_t blk = sh / BS;
    const int c0 = static_cast<int>(sh - blk * BS);
    const int64_t tf = t0 - 1 + i;
    const int c1 = c0 + len;

    // Runs that touch every 16-byte column group of the block row go through
    // LDS (whole-line traffic on both sides); shorter runs use lane tiles
    // that load or store only the column groups they cover.
    if (c0 < CG && c1 > BS - CG) {
      staged_run<ELT_C, ELT_L, CODEC, LDT, BS, SCATTER>(a, cache + blk * a.nrows * BS * ELT_C,
                                                        lin + tf * a.lin_token_stride, c0, c1, kv, layer, lds,
                                                        r_begin, r_end, static_cast<int>(tile & 0xFFFF));
      continue;
    }

    const int j0 = c0 / CG;
    const int j1 = (c1 - 1) / CG;
    for (int g = static_cast<int>(r_begin / RPL) + lane; g < ngroups; g += kWave) {
      const int64_t r0 = static_cast<int64_t>(g) * RPL;
      float sc = 1.0f;
      if constexpr (CODEC != kCopy) sc = load_scale(a, kv, layer, r0 / a.head_dim);
      uint8_t* const crow = cache + (blk * a.nrows + r0) * BS * ELT_C;
      uint8_t* const lrow = lin + tf * a.lin_token_stride + r0 * ELT_L;
      // One 16-byte column group at a time keeps the register tile at RPL
      // (gather) or CG (scatter) vectors.
#pragma unroll 1
      for (int j = j0; j <= j1; ++j) {
        const int lo = j * CG;
        uint8_t* const cgrp = crow + lo * ELT_C;
        if constexpr (!SCATTER) {
          u32x4 d[RPL];
#pragma unroll
          for (int q = 0; q < RPL; ++q) d[q] = ld16_cached(cgrp + q * BS * ELT_C);
#pragma unroll
          for (int cc = 0; cc < CG; ++cc) {
            const int c = lo + cc;
            if (c >= c0 && c < c1)
              st16(lrow + static_cast<int64_t>(c - c0) * a.lin_token_stride,
                   gather_column<ELT_C, ELT_L, CODEC, LDT, RPL>(d, cc, sc));
          }
        } else {
          u32x4 in[CG];
#pragma unroll
          for (int cc = 0; cc < CG; ++cc) {
            const int c = lo + cc;
            in[cc] = u32x4{0u, 0u, 0u, 0u};
            if (c >= c0 && c < c1) in[cc] = ld16(lrow + static_cast<int64_t>(c - c0) * a.lin_token_stride);
          }
          if (lo >= c0 && lo + CG <= c1) {
            encode_tile<ELT_C, ELT_L, CODEC, LDT, CG, RPL>(
                in, sc, [&](int q, const u32x4& row) { st16_cached(cgrp + q * BS * ELT_C, row); });
          } else {
#pragma unroll
            for (int q = 0; q < RPL; ++q) {
#pragma unroll
              for (int cc = 0; cc < CG; ++cc) {
                const int c = lo + cc;
                if (c >= c0 && c < c1)
                  store_elem<ELT_C>(cgrp + (q * BS + cc) * ELT_C,
                                    scatter_elem<ELT_C, ELT_L, CODEC, LDT>(in[cc], q, sc));
              }
            }
          }
        }
      }
    }
  }

  if constexpr (!SCATTER) {
    if (a.fill_zeros) {
      uint64_t skipped = ~vmask & window;
      const int64_t row_bytes = r_end * ELT_L;
      const u32x4 zero = {0u, 0u, 0u, 0u};
      while (skipped) {
        const int i = __builtin_ctzll(skipped);
        skipped &= skipped - 1;
        uint8_t* const row = lin + (t0 - 1 + i) * a.lin_token_stride;
        for (int64_t k = r_begin * ELT_L + static_cast<int64_t>(lane) * 16; k < row_bytes; k += kWave * 16)
          st16(row + k, zero);
      }
    }
  }
}

// ----- generic element-wise kernel (any block size / alignment) ----------------

template <int ELT>
__device__ __forceinline__ uint32_t load_elem(const uint8_t* p) {
  if constexpr (ELT == 1) return *p;
  else if constexpr (ELT == 2) return *reinterpret_cast<const uint16_t*>(p);
  else return *reinterpret_cast<const uint32_t*>(p);
}

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
    const int64_t s = a.slots[t];
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

constexpr int kChunksPerSplit = 1;

template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS, bool SCATTER>
hipError_t launch_tile(const TileArgs& a_in, int64_t planes, hipStream_t stream) {
  constexpr int RPL = 16 / ELT_L;
  constexpr int NCG = BS / (16 / ELT_C);
  constexpr int64_t kChunkRows = (kWave / NCG) * RPL;
  TileArgs a = a_in;
  a.split_rows = kChunkRows * kChunksPerSplit;
  const int64_t splits = (a.nrows + a.split_rows - 1) / a.split_rows;
  if (splits > 65535) return hipErrorInvalidValue;
  const int64_t tiles = (a.num_tokens + kTileTokens - 1) / kTileTokens;
  const int64_t blocks = (tiles + kWavesPerBlock - 1) / kWavesPerBlock;
  hipLaunchKernelGGL((paged_tile_kernel<ELT_C, ELT_L, CODEC, LDT, BS, SCATTER>),
                     dim3(static_cast<uint32_t>(blocks), static_cast<uint32_t>(planes), static_cast<uint32_t>(splits)),
                     dim3(kBlockThreads), 0, stream, a);
  return hipGetLastError();
}

template <int ELT_C, int ELT_L, int CODEC, int LDT, bool SCATTER>
hipError_t dispatch_bs(const TileArgs& a, int64_t bs, bool fast, int64_t planes, hipStream_t stream) {
  if (fast) {
    if constexpr (ELT_C != 1) {
      if (bs == 8) return launch_tile<ELT_C, ELT_L, CODEC, LDT, 8, SCATTER>(a, planes, stream);
    }
    if (bs == 16) return launch_tile<ELT_C, ELT_L, CODEC, LDT, 16, SCATTER>(a, planes, stream);
    if (bs == 32) return launch_tile<ELT_C, ELT_L, CODEC, LDT, 32, SCATTER>(a, planes, stream);
  }
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
  a.block_size = static_cast<int32_t>(p.block_size);

  const int rpl = 16 / p.lin_elt;
  const int cg = 16 / p.cache_elt;
  bool fast = (p.head_dim % rpl == 0) && (p.lin_token_stride % 16 == 0) && (p.lin_layer_stride % 16 == 0) &&
              (p.block_size % cg == 0);
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
