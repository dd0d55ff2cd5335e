// Access-pattern ceiling of a paged copy on MI355X (gfx950): whole blocks
// copied between two block-addressed regions in a caller-given block order,
// with no index resolution, transpose or arithmetic.  A paged gather reads
// its cache blocks in the order the slot mapping visits them and writes the
// linear side in order; a paged scatter does the reverse; the FP8 codecs read
// two bytes per byte written (quant-store) or one per two (dequant-gather).
// Timing this kernel on the caller's own buffers, with the caller's own block
// order, gives the rate that order allows a pure copy: the bound the paged
// kernels are measured against.
//
// Shape: one wave per unit of 1 KiB on the narrower side (one 16-byte vector
// per lane), 2 KiB (two vectors per lane) on the wider side when the sides
// differ; every wave instruction covers 1 KiB contiguous, each wave does one
// unit and exits (the copy shape that measures fastest on this GPU).  Stores
// are non-temporal, or with write_through also agent-scope (through the
// issuing XCD's L2, like the paged gathers' linear stores); bench.py times
// both and takes the faster as the ceiling.
#include "kv_hip_common.h"
#include "kv_launch.h"

namespace kvhip {

// RV / WV: 16-byte vectors per lane read / written (1:1, 2:1 or 1:2); STP:
// cache-policy bits of the stores.
template <int RV, int WV, int STP>
__global__ __launch_bounds__(kBlockThreads) void block_pattern_kernel(const uint8_t* __restrict__ src,
                                                                      uint8_t* __restrict__ dst,
                                                                      const int32_t* __restrict__ src_blocks,
                                                                      const int32_t* __restrict__ dst_blocks,
                                                                      int64_t num_units, int32_t units_per_block,
                                                                      int64_t src_region_blocks,
                                                                      int64_t dst_region_blocks,
                                                                      int64_t src_block_bytes, int64_t dst_block_bytes,
                                                                      int64_t src_plane_stride,
                                                                      int64_t dst_plane_stride) {
  // Wave-uniform unit index, so the block ids, bases and the store descriptor stay in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int64_t unit = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + wave;
  if (unit >= num_units) return;
  const int lane = lane_id();
  const int64_t plane = blockIdx.y;
  // 32-bit division (the launcher keeps num_units below 2^32): a 64-bit one
  // costs each short-lived wave hundreds of scalar cycles.
  const uint32_t u32 = static_cast<uint32_t>(unit);
  const uint32_t upb = static_cast<uint32_t>(units_per_block);
  const int64_t blk = u32 / upb;
  const int64_t in = u32 - static_cast<uint32_t>(blk) * upb;
  const int64_t sb = src_blocks != nullptr ? src_blocks[blk] : blk;
  const int64_t db = dst_blocks != nullptr ? dst_blocks[blk] : blk;
  if (sb < 0 || sb >= src_region_blocks || db < 0 || db >= dst_region_blocks) return;
  const uint8_t* s = src + plane * src_plane_stride + sb * src_block_bytes + in * (RV * 1024) + lane * 16;
  // The unit's destination (wave-uniform) as a buffer, the lane's piece as its offset.
  const buf_t d = make_buf(dst + plane * dst_plane_stride + db * dst_block_bytes + in * (WV * 1024));
  const uint32_t off = static_cast<uint32_t>(lane) * 16u;
  u32x4 v[RV];
#pragma unroll
  for (int k = 0; k < RV; ++k) v[k] = ld16(s + k * 1024);
  if constexpr (RV == 2 && WV == 1) {
    buf_st16_p<STP>(d, off, v[0] ^ v[1]);
  } else {
#pragma unroll
    for (int k = 0; k < WV; ++k) buf_st16_p<STP>(d, off + k * 1024u, v[0]);
  }
}

hipError_t launch_block_pattern(const BlockPatternParams& p, hipStream_t stream) {
  if (p.num_blocks <= 0 || p.planes <= 0) return hipSuccess;
  if (p.src == nullptr || p.dst == nullptr || p.planes > 65535 || p.src_block_bytes <= 0 ||
      p.dst_block_bytes <= 0 || p.src_block_bytes % 1024 != 0 || p.dst_block_bytes % 1024 != 0)
    return hipErrorInvalidValue;
  int rv = 1, wv = 1;
  if (p.src_block_bytes == 2 * p.dst_block_bytes) rv = 2;
  else if (p.dst_block_bytes == 2 * p.src_block_bytes) wv = 2;
  else if (p.src_block_bytes != p.dst_block_bytes) return hipErrorInvalidValue;
  const int64_t upb = p.src_block_bytes / (rv * 1024);
  const int64_t units = p.num_blocks * upb;
  const int64_t groups = (units + kWavesPerBlock - 1) / kWavesPerBlock;
  if (upb > 0x7FFFFFFF || units > int64_t{0xFFFFFFFF}) return hipErrorInvalidValue;
  const dim3 grid(static_cast<uint32_t>(groups), static_cast<uint32_t>(p.planes));
  const auto* s = static_cast<const uint8_t*>(p.src);
  auto* d = static_cast<uint8_t*>(p.dst);
  const int32_t upb32 = static_cast<int32_t>(upb);
  auto launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, grid, dim3(kBlockThreads), 0, stream, s, d, p.src_blocks, p.dst_blocks, units, upb32,
                       p.src_region_blocks, p.dst_region_blocks, p.src_block_bytes, p.dst_block_bytes,
                       p.src_plane_stride, p.dst_plane_stride);
  };
  if (p.write_through) {
    if (rv == 2) launch(block_pattern_kernel<2, 1, kBufWT>);
    else if (wv == 2) launch(block_pattern_kernel<1, 2, kBufWT>);
    else launch(block_pattern_kernel<1, 1, kBufWT>);
  } else {
    if (rv == 2) launch(block_pattern_kernel<2, 1, kBufNT>);
    else if (wv == 2) launch(block_pattern_kernel<1, 2, kBufNT>);
    else launch(block_pattern_kernel<1, 1, kBufNT>);
  }
  return hipGetLastError();
}

}  // namespace kvhip
