// Kernel arguments and element helpers shared by the paged-A tile kernels
// (kv_paged_tiles.hip: workgroup-cooperative kernel, generic element kernel;
// kv_paged_waves.hip: per-wave gather kernel).
#pragma once

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
  int32_t owner_exclusive;     // every tag of `epoch` in owner was claimed by this call
  int32_t block_size;          // used by the generic kernel only
  float inv_head_dim;          // 1 / head_dim, for small-integer division by head_dim
  BlockTableSlots bt;          // block_tables set: slots derived per dense token
  int32_t row_groups;          // tile kernel: row groups per block (grid x of a gather = tile * row_groups + group)
  int32_t scan_dupes;          // scatter: resolve repeated slots with a ScanTable instead of claim tags
};

// Slot of token t: the slot vector's entry, or the block-table slot of the
// dense token t.
__device__ __forceinline__ int64_t slot_at(const TileArgs& a, int64_t t) {
  if (a.bt.block_tables != nullptr) return block_table_slot(a.bt, t);
  return a.slots[t];
}

constexpr int kTileTokens = 16;

// Small scatters resolve repeated destinations without the claim pass (one
// launch and one dependent load fewer): every workgroup maps each slot of the
// call to the last token that writes it, in LDS -- open addressing over
// 2 x kScanTokens entries, a 64-bit compare-and-swap claiming an entry for the
// slot and an atomic max keeping the token -- and a token writes only if it is
// its slot's last token, the claim pass's rule (last writer wins).  The host
// keeps such calls at or below kScanTokens tokens, so at most half the
// entries are taken and every probe sequence ends.
constexpr int kScanEntries = 2 * kScanTokens;
constexpr unsigned long long kScanEmpty = ~0ull;

struct ScanTable {
  unsigned long long key[kScanEntries];
  int last[kScanEntries];
};

// The workgroup's table (static LDS of the kernels that call it).
__device__ __forceinline__ ScanTable& scan_table() {
  __shared__ ScanTable tb;
  return tb;
}

__device__ __forceinline__ uint32_t scan_hash(int64_t s) {
  return static_cast<uint32_t>((static_cast<uint64_t>(s) * 0x9E3779B97F4A7C15ull) >> 40) & (kScanEntries - 1);
}

// Fills the table from the call's slots; every thread of the workgroup calls
// it (it holds two workgroup barriers).
template <int NT>
__device__ void scan_build(ScanTable& tb, const TileArgs& a) {
  const int tid = static_cast<int>(threadIdx.x);
  for (int e = tid; e < kScanEntries; e += NT) {
    tb.key[e] = kScanEmpty;
    tb.last[e] = -1;
  }
  __syncthreads();
  for (int64_t j = tid; j < a.num_tokens; j += NT) {
    const int64_t s = slot_at(a, j);
    if (s < 0 || s >= a.num_slots) continue;
    uint32_t h = scan_hash(s);
    for (int probe = 0; probe < kScanEntries; ++probe) {
      const unsigned long long prev = atomicCAS(&tb.key[h], kScanEmpty, static_cast<unsigned long long>(s));
      if (prev == kScanEmpty || prev == static_cast<unsigned long long>(s)) {
        atomicMax(&tb.last[h], static_cast<int>(j));
        break;
      }
      h = (h + 1) & (kScanEntries - 1);
    }
  }
  __syncthreads();
}

// True when token t is the last token of the call writing slot s (s valid).
__device__ __forceinline__ bool scan_is_last(const ScanTable& tb, int64_t s, int64_t t) {
  uint32_t h = scan_hash(s);
  for (int probe = 0; probe < kScanEntries; ++probe) {
    const unsigned long long k = tb.key[h];
    if (k == static_cast<unsigned long long>(s)) return tb.last[h] == static_cast<int>(t);
    if (k == kScanEmpty) return false;
    h = (h + 1) & (kScanEntries - 1);
  }
  return false;
}

// head = row / head_dim for rows below 2^24: a float reciprocal and one
// exact correction step.
__device__ __forceinline__ int head_of_row(const TileArgs& a, int row) {
  const int hd = static_cast<int>(a.head_dim);
  int head = static_cast<int>(static_cast<float>(row) * a.inv_head_dim);
  if (head * hd > row) --head;
  else if ((head + 1) * hd <= row) ++head;
  return head;
}

__device__ __forceinline__ float load_scale(const TileArgs& a, int kv, int layer, int64_t head) {
  const float* s = a.scale[kv];
  if (a.scale_mode == 0) return s[0];
  if (a.scale_mode == 1) return s[head];
  return s[static_cast<int64_t>(layer) * a.num_heads + head];
}

template <int ELT>
__device__ __forceinline__ void store_elem(uint8_t* p, uint32_t v) {
  if constexpr (ELT == 1) *p = static_cast<uint8_t>(v);
  else if constexpr (ELT == 2) *reinterpret_cast<uint16_t*>(p) = static_cast<uint16_t>(v);
  else *reinterpret_cast<uint32_t*>(p) = v;
}

template <int ELT>
__device__ __forceinline__ uint32_t load_elem(const uint8_t* p) {
  if constexpr (ELT == 1) return *p;
  else if constexpr (ELT == 2) return *reinterpret_cast<const uint16_t*>(p);
  else return *reinterpret_cast<const uint32_t*>(p);
}

// Element `idx` of a 16-byte piece holding ELT-byte elements.
template <int ELT>
__device__ __forceinline__ uint32_t piece_elem(const u32x4& v, int idx) {
  if constexpr (ELT == 1) return elem8(v, idx);
  else if constexpr (ELT == 2) return elem16(v, idx);
  else return v[idx];
}

// Per-wave LDS-staged gather (kv_paged_waves.hip), used for the FP8
// dequant-gather: its in-register 8x16 byte transposes need an eighth of the
// LDS instructions of the cooperative kernel's column reads.
template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS>
hipError_t launch_wave_gather(const TileArgs& a, int64_t planes, hipStream_t stream);

// Per-wave linear -> paged FP8 quant-store (kv_paged_waves.hip): the
// converter packs four tokens of one cache row per dword, so the quantised
// tile leaves the lane already transposed.
template <int ELT_C, int ELT_L, int CODEC, int LDT, int BS>
hipError_t launch_wave_scatter(const TileArgs& a, int64_t planes, hipStream_t stream);

// Per-wave 16-bit linear -> paged scatter in destination order
// (kv_paged_waves.hip): needs this call's claim tags as the inverse map.
template <int BS>
hipError_t launch_wave_copy_scatter(const TileArgs& a, int64_t planes, hipStream_t stream);

}  // namespace kvhip
