// Host-side launcher interfaces shared by the kernel translation units and
// the C-ABI layer.  Nothing here is exported from the shared library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kv_hip_common.h"

namespace kvhip {

constexpr int kMaxPlanes = 128;

// Paged scatters of at most this many tokens resolve repeated slots inside
// their kernel (PagedTileParams::scan_dupes) instead of a claim pass.
constexpr int kScanTokens = 256;

// Paged-A layout [NL, NB, NH, HD, BS] (block_size innermost) <-> token-major
// linear rows.  K and V are the two planes of every layer.
struct PagedTileParams {
  int scatter;         // 0: paged -> linear (gather), 1: linear -> paged (scatter)
  int codec;           // Codec: copy, fp8 e4m3, fp8 e5m2
  int cache_elt;       // bytes per cache element (1 for fp8 codecs)
  int lin_elt;         // bytes per linear element
  int lin_dtype;       // LinDtype, used by the fp8 codecs
  void* cache[2];      // K, V caches (layer 0)
  void* lin[2];        // K, V linear bases (layer 0, token 0)
  const int64_t* slots;
  int64_t num_layers;
  int64_t num_tokens;
  int64_t num_blocks;
  int64_t num_heads;
  int64_t head_dim;
  int64_t block_size;
  int64_t lin_token_stride;  // bytes
  int64_t lin_layer_stride;  // bytes
  const float* scale[2];
  int scale_mode;            // 0 scalar, 1 [NH], 2 [NL, NH]
  int fill_zeros;            // gather: write zeros for skipped tokens
  const uint64_t* owner;     // scatter claim tags (nullable)
  uint32_t epoch;
  // The tags of `epoch` in owner are exactly this call's claims (an epoch no
  // earlier call on the array used), so owner is the call's inverse map; false
  // after a reset-and-claim pass, which leaves earlier calls' tags of the same
  // epoch on slots this call does not write.
  int owner_exclusive;
  BlockTableSlots bt;        // block_tables set: slots derived per dense token, `slots` unused
  // Scatter of at most kScanTokens tokens without claim tags: the kernels find
  // each slot's last token themselves (ScanTable).  launch_paged_tiles returns
  // hipErrorNotSupported, launching nothing, when the call's kernel cannot.
  int scan_dupes;
};

hipError_t launch_paged_tiles(const PagedTileParams& p, hipStream_t stream);

// Row copies between two row-addressed planes: token-major caches
// ([NB, BS, ...] slot rows), linear buffers and opaque byte rows.  Either side
// is addressed directly (row = token + offset) or through an index vector.
struct RowCopyParams {
  const uint64_t* src_planes;   // host array (nullable when src_table is set)
  const uint64_t* dst_planes;
  const uint64_t* src_table;    // device array of plane bases (nullable)
  const uint64_t* dst_table;
  int64_t num_planes;
  const int64_t* src_idx;       // device (nullable => direct)
  const int64_t* dst_idx;
  int64_t num_tokens;           // index entries
  int64_t num_rows_out;         // >= num_tokens for a direct, zero-filled tail
  int64_t src_offset;
  int64_t dst_offset;
  int64_t src_rows;             // valid row range of each side
  int64_t dst_rows;
  int64_t row_bytes;
  int64_t src_stride;           // bytes between rows
  int64_t dst_stride;
  int zero_invalid;             // direct destination: zero rows whose source is skipped
  const uint64_t* owner;        // claim tags over destination rows (nullable)
  uint32_t epoch;
  int owner_exclusive;          // the tags of `epoch` are exactly this call's claims (see PagedTileParams)
  // CSR source addressing (nullable): token u = b * dense_len + pos reads
  // row src_idx[src_indptr[b] + pos]; src_idx holds index_count entries.
  const int64_t* src_indptr;
  int64_t dense_len;
  int64_t index_count;
  int64_t idx_stride;           // elements between index entries (0 or 1: packed vectors)
  // Paged row addressing (page_rows > 0): row r of a side sits at byte
  // (r / page_rows) * page_stride + (r % page_rows) * stride of its plane;
  // 0 keeps the plain r * stride.
  int64_t src_page_rows;
  int64_t src_page_stride;
  int64_t dst_page_rows;
  int64_t dst_page_stride;
};

hipError_t launch_row_copy(const RowCopyParams& p, hipStream_t stream);

// Destinations of a scatter for the claim pass: token i targets idx[i *
// idx_stride] (or the block-table slot of dense token i when bt.block_tables
// is set); with src_idx set, a token whose source src_idx[i * idx_stride]
// lies outside [0, src_rows) writes nothing and claims nothing.
struct ClaimSource {
  const int64_t* idx = nullptr;
  int64_t idx_stride = 1;
  BlockTableSlots bt{};
  const int64_t* src_idx = nullptr;
  int64_t src_rows = 0;
};

// Marks, for every destination row, the last token (in token order) that
// writes it.  With `reset` it instead zeroes the entries of the rows the
// tokens write, so that a following claim pass needs no cleared array.
hipError_t launch_claim(const ClaimSource& src, int64_t n, int64_t rows, uint64_t* owner, uint32_t epoch,
                        hipStream_t stream, bool reset = false);
hipError_t launch_fill_u64(uint64_t* p, int64_t n, uint64_t value, hipStream_t stream);

// Maxima of idx[0, n) per workgroup into partial[0, parts), then `stamp`
// into partial[parts, 2 * parts) (kv_rows.hip).
hipError_t launch_index_max(const int64_t* idx, int64_t n, int64_t* partial, int64_t parts, int64_t stamp,
                            hipStream_t stream);

// Block-granular byte copies between an LMCache staging object and padded pages.
struct StridedBlockParams {
  uint8_t* staging;
  const uint64_t* paged_ptrs;   // host array, num_layers entries
  const int64_t* block_ids;
  int64_t direction;            // 0: staging -> pages, 1: pages -> staging
  int64_t num_layers;
  int64_t idx_start;
  int64_t n_valid;
  int64_t offset_in_object;
  int64_t staging_tokens;
  int64_t block_size;
  int64_t row_bytes;
  int64_t paged_block_stride;
  int64_t mode;                 // 0 plain rows, 1 values block then scales block
  int64_t value_bytes;
  int64_t scale_bytes;
};

hipError_t launch_strided_blocks(const StridedBlockParams& p, hipStream_t stream);

// Byte ranges copied by one launch each (count may exceed it: several launches).
constexpr int kBatchCopyMax = 96;

// Copies `count` byte ranges src[i] -> dst[i] of size[i] bytes, all addresses
// device-visible (device memory or the device mapping of pinned host memory),
// on at most `max_groups` workgroups per launch (0: one per 64 KiB tile).
hipError_t launch_batch_copy(const uint64_t* src, const uint64_t* dst, const uint64_t* size, int64_t count,
                             uint32_t max_groups, hipStream_t stream);
// Per-tile descriptors for batches larger than kBatchCopyMax ranges: the
// number of 64 KiB tiles of the ranges, the (src, dst, bytes) triple of each
// tile written into host memory `desc` (3 values per tile), and one launch
// over descriptors that the device reads at `desc` (a pinned, mapped copy).
uint64_t batch_copy_tile_count(const uint64_t* size, int64_t count);
void batch_copy_fill_desc(const uint64_t* src, const uint64_t* dst, const uint64_t* size, int64_t count,
                          uint64_t* desc);
hipError_t launch_batch_copy_desc(const uint64_t* desc, uint64_t tiles, uint32_t max_groups, hipStream_t stream);

// Whole blocks copied between two block-addressed regions of `planes` planes
// in a given block order (the access-pattern ceiling of a paged copy):
// block i of the copy reads block src_blocks[i] (or i) of the source and
// writes block dst_blocks[i] (or i) of the destination.  Block sizes are
// multiples of 1 KiB, equal or in a 2:1 / 1:2 ratio; block ids outside
// [0, *_region_blocks) are skipped.
struct BlockPatternParams {
  const void* src;
  void* dst;
  const int32_t* src_blocks;
  const int32_t* dst_blocks;
  int64_t num_blocks;
  int64_t src_region_blocks;
  int64_t dst_region_blocks;
  int64_t src_block_bytes;
  int64_t dst_block_bytes;
  int64_t planes;
  int64_t src_plane_stride;  // bytes
  int64_t dst_plane_stride;
  int write_through;         // 1: agent-scope stores (through the L2), 0: non-temporal only
};

hipError_t launch_block_pattern(const BlockPatternParams& p, hipStream_t stream);

// ----- CacheGen-style uniform-bin codec ------------------------------------------------

// Input element types of the encoder.
enum CacheGenInput : int { kCgF32 = 0, kCgF16 = 1, kCgBF16 = 2, kCgF64 = 3 };

// Device workspace the encoder needs (per-workgroup ranges and the bin counters).
constexpr int64_t kCacheGenWorkspaceBytes = 16384;

// Bins of the `n` elements of `x` over their own [min, max] (torch-path rounding, or the
// reference kernel's when `native`; float32 input only), the codebook[num_bins] and the
// cdf[num_bins + 1]; three launches, no host synchronisation.
hipError_t launch_cachegen_encode(const void* x, int in_dtype, int64_t n, int num_bins, bool native, uint8_t* enc,
                                  float* codebook, float* cdf, void* workspace, hipStream_t stream);

// Bins of float32 `x` with a caller-given minimum and scale, the reference kernel's rounding.
hipError_t launch_cachegen_bins(const float* x, uint8_t* enc, float min_val, float scale, int64_t n, int num_bins,
                                hipStream_t stream);

// out[i] = table[codes[i]] for entries of `elem_bytes` (1, 2, 4, 8 or 16) bytes.  With
// table_len in [1, 255] codes at or past the end read zeros and the largest such code is
// stored to *max_code (atomic max; the caller clears it); table_len < 0 reads a float32
// table of unknown length straight from global memory (no check).
hipError_t launch_cachegen_decode(const uint8_t* codes, int64_t n, const void* table, int table_len, int elem_bytes,
                                  void* out, int32_t* max_code, hipStream_t stream);

}  // namespace kvhip
