// Kernel arguments and element helpers shared by the paged-A tile kernels
// (kv_paged_tiles.hip: workgroup-cooperative kernel, generic element kernel;
// kv_paged_waves.hip: per-wave gather kernel).
#pragma once

#include "kv_hip_common.h"

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
};

// Slot of token t: the slot vector's entry, or the block-table slot of the
// dense token t.
__device__ __forceinline__ int64_t slot_at(const TileArgs& a, int64_t t) {
  if (a.bt.block_tables != nullptr) return block_table_slot(a.bt, t);
  return a.slots[t];
}

constexpr int kTileTokens = 16;

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
