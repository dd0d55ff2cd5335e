// Batched host <-> device byte copies for MI355X (gfx950): the LMCache staging
// step on the far side of the KV buffers.
//
// Every range is cut into 64 KiB tiles and workgroups stride over the tiles,
// so a batch of many small chunks costs one launch instead of one runtime
// call per chunk.  Up to kBatchCopyMax ranges travel in the kernel arguments
// (a workgroup finds a tile's range from the tile prefix there); larger
// batches use one descriptor per tile in pinned host memory.  The
// grid holds at most `max_groups` workgroups: the host link needs far fewer
// requests in flight than the chip can issue, and a small grid also leaves
// the other compute units to concurrent kernels.  The host side of every
// range is pinned host memory addressed through its device mapping, so the
// loads or stores of that side travel over the host link; the access width is
// the widest power of two (<= 16 bytes) to which source and destination are
// equally aligned, with byte-wise heads and tails.  Each thread keeps four
// vectors in flight to cover the link latency.
#include "kv_hip_common.h"
#include "kv_launch.h"

namespace kvhip {

namespace {

constexpr uint32_t kTileBytes = 64u << 10;
constexpr int kInflight = 4;

struct BatchCopyArgs {
  uint64_t src[kBatchCopyMax];
  uint64_t dst[kBatchCopyMax];
  uint64_t size[kBatchCopyMax];
  uint32_t tile_end[kBatchCopyMax];  // inclusive prefix of tiles per range
  int32_t count;
};

template <int VEC>
__device__ __forceinline__ void copy_tile(const uint8_t* s, uint8_t* d, uint32_t n) {
  using V = typename VecType<VEC>::T;
  const uint32_t tid = threadIdx.x;
  uint32_t head = static_cast<uint32_t>((VEC - (reinterpret_cast<uintptr_t>(d) & (VEC - 1))) & (VEC - 1));
  if (head > n) head = n;
  for (uint32_t i = tid; i < head; i += kBlockThreads) d[i] = s[i];
  const uint32_t body = (n - head) / VEC;
  const uint8_t* sb = s + head;
  uint8_t* db = d + head;
  uint32_t i = tid;
  for (; i + (kInflight - 1) * kBlockThreads < body; i += kInflight * kBlockThreads) {
    V v[kInflight];
#pragma unroll
    for (int k = 0; k < kInflight; ++k) v[k] = ldv<VEC>(sb + static_cast<size_t>(i + k * kBlockThreads) * VEC);
#pragma unroll
    for (int k = 0; k < kInflight; ++k) stv<VEC>(db + static_cast<size_t>(i + k * kBlockThreads) * VEC, v[k]);
  }
  for (; i < body; i += kBlockThreads) stv<VEC>(db + static_cast<size_t>(i) * VEC, ldv<VEC>(sb + static_cast<size_t>(i) * VEC));
  for (uint32_t t = head + body * VEC + tid; t < n; t += kBlockThreads) d[t] = s[t];
}

// Copies n bytes at the widest access to which source and destination are equally aligned.
__device__ __forceinline__ void copy_range(uint64_t src, uint64_t dst, uint32_t n) {
  const uint8_t* s = reinterpret_cast<const uint8_t*>(src);
  uint8_t* d = reinterpret_cast<uint8_t*>(dst);
  const uint32_t rel = static_cast<uint32_t>((src ^ dst) & 15u);
  if (rel == 0) copy_tile<16>(s, d, n);
  else if ((rel & 7u) == 0) copy_tile<8>(s, d, n);
  else if ((rel & 3u) == 0) copy_tile<4>(s, d, n);
  else if ((rel & 1u) == 0) copy_tile<2>(s, d, n);
  else copy_tile<1>(s, d, n);
}

// One (src, dst, bytes) descriptor per tile, read from pinned host memory
// through its device mapping.  A workgroup loads the descriptor of its next
// tile before copying the current one, so the read's link latency overlaps
// the copy.  The grid never exceeds `tiles`.
__global__ __launch_bounds__(kBlockThreads) void batch_copy_desc_kernel(const uint64_t* desc, uint32_t tiles) {
  uint32_t tile = blockIdx.x;
  uint64_t s = desc[3 * static_cast<uint64_t>(tile)];
  uint64_t d = desc[3 * static_cast<uint64_t>(tile) + 1];
  uint64_t n = desc[3 * static_cast<uint64_t>(tile) + 2];
  while (true) {
    const uint32_t next = tile + gridDim.x;
    uint64_t ns = 0, nd = 0, nn = 0;
    if (next < tiles) {
      ns = desc[3 * static_cast<uint64_t>(next)];
      nd = desc[3 * static_cast<uint64_t>(next) + 1];
      nn = desc[3 * static_cast<uint64_t>(next) + 2];
    }
    copy_range(s, d, static_cast<uint32_t>(n));
    if (next >= tiles) break;
    tile = next;
    s = ns;
    d = nd;
    n = nn;
  }
}

__global__ __launch_bounds__(kBlockThreads) void batch_copy_kernel(const BatchCopyArgs a) {
  const uint32_t tiles = a.tile_end[a.count - 1];
  for (uint32_t tile = blockIdx.x; tile < tiles; tile += gridDim.x) {
    // Range of this tile: the first whose inclusive tile prefix exceeds it (uniform per block).
    int lo = 0, hi = a.count - 1;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (a.tile_end[mid] > tile) hi = mid;
      else lo = mid + 1;
    }
    const uint32_t first = lo == 0 ? 0u : a.tile_end[lo - 1];
    const uint64_t off = static_cast<uint64_t>(tile - first) * kTileBytes;
    const uint64_t left = a.size[lo] - off;
    const uint32_t n = static_cast<uint32_t>(left < kTileBytes ? left : kTileBytes);
    copy_range(a.src[lo] + off, a.dst[lo] + off, n);
  }
}

}  // namespace

uint64_t batch_copy_tile_count(const uint64_t* size, int64_t count) {
  uint64_t tiles = 0;
  for (int64_t i = 0; i < count; ++i) tiles += (size[i] + kTileBytes - 1) / kTileBytes;
  return tiles;
}

void batch_copy_fill_desc(const uint64_t* src, const uint64_t* dst, const uint64_t* size, int64_t count,
                          uint64_t* desc) {
  for (int64_t i = 0; i < count; ++i) {
    for (uint64_t off = 0; off < size[i]; off += kTileBytes) {
      const uint64_t left = size[i] - off;
      desc[0] = src[i] + off;
      desc[1] = dst[i] + off;
      desc[2] = left < kTileBytes ? left : kTileBytes;
      desc += 3;
    }
  }
}

hipError_t launch_batch_copy_desc(const uint64_t* desc, uint64_t tiles, uint32_t max_groups, hipStream_t stream) {
  if (tiles == 0) return hipSuccess;
  if (desc == nullptr || tiles > 0x7FFFFFFFu) return hipErrorInvalidValue;
  const uint32_t groups = (max_groups != 0 && tiles > max_groups) ? max_groups : static_cast<uint32_t>(tiles);
  hipLaunchKernelGGL(batch_copy_desc_kernel, dim3(groups), dim3(kBlockThreads), 0, stream, desc,
                     static_cast<uint32_t>(tiles));
  return hipGetLastError();
}

hipError_t launch_batch_copy(const uint64_t* src, const uint64_t* dst, const uint64_t* size, int64_t count,
                             uint32_t max_groups, hipStream_t stream) {
  for (int64_t base = 0; base < count; base += kBatchCopyMax) {
    const int64_t n = (count - base) < kBatchCopyMax ? (count - base) : kBatchCopyMax;
    BatchCopyArgs a{};
    uint64_t tiles = 0;
    int32_t m = 0;
    for (int64_t i = 0; i < n; ++i) {
      const uint64_t bytes = size[base + i];
      if (bytes == 0) continue;
      tiles += (bytes + kTileBytes - 1) / kTileBytes;
      if (tiles > 0x7FFFFFFFu) return hipErrorInvalidValue;
      a.src[m] = src[base + i];
      a.dst[m] = dst[base + i];
      a.size[m] = bytes;
      a.tile_end[m] = static_cast<uint32_t>(tiles);
      ++m;
    }
    if (m == 0) continue;
    a.count = m;
    const uint32_t groups = (max_groups != 0 && tiles > max_groups) ? max_groups : static_cast<uint32_t>(tiles);
    hipLaunchKernelGGL(batch_copy_kernel, dim3(groups), dim3(kBlockThreads), 0, stream, a);
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

}  // namespace kvhip
