// Row-granular KV transfers for MI355X (gfx950).
//
// Every token-major layout of the path reduces to "copy one row of R bytes
// per (plane, token)": SGLang-MP split caches [NB, BS, NH, HS] <-> LMCache
// [2, NL, T, NH*HS] buffers, the per-layer list and legacy 6-D caches, the
// MLA latent rows [NB, BS, D], the opaque DSV4 byte rows, whole paged blocks
// and SGLang HiCache items (one (page, layer) row of a layer-first or
// page-first pool).  One side of the copy is indexed by a slot/row vector (or
// both); slot < 0 skips the token.  A side may also be paged: row r then sits
// at (r / page_rows) * page_stride + (r % page_rows) * stride.
//
// Rows are cut into VEC-byte pieces (VEC = the widest power of two dividing
// the row size, strides and plane bases); one block moves 512 consecutive
// pieces of the flattened (token, piece) range of one plane (grid y = plane),
// two per thread, whatever the row size: a short row shares a block with its
// neighbours, a long one spans several blocks.  Each wave keeps only two
// vectors per lane in flight, the access shape that reaches the highest HBM
// copy rate on MI355X, and the block resolves the indices of the rows it
// touches once, into LDS, before streaming.  Skipped tokens of a directly
// addressed destination are zero filled; an indexed destination can be
// protected by claim tags so duplicate slots keep last-writer-wins.
#include "kv_hip_common.h"
#include "kv_launch.h"

namespace kvhip {

struct RowArgs {
  uint64_t src_planes[kMaxPlanes];
  uint64_t dst_planes[kMaxPlanes];
  const uint64_t* src_table;
  const uint64_t* dst_table;
  const int64_t* src_idx;
  const int64_t* dst_idx;
  const uint64_t* owner;
  int64_t num_tokens;
  int64_t num_rows_out;
  int64_t src_offset;
  int64_t dst_offset;
  int64_t src_rows;
  int64_t dst_rows;
  int64_t row_bytes;
  int64_t src_stride;
  int64_t dst_stride;
  int32_t plane_base;       // first plane of this launch in the table arrays
  int32_t num_planes;       // planes in this launch
  int32_t zero_invalid;
  uint32_t epoch;
  const int64_t* src_indptr;  // CSR source addressing (nullable)
  uint32_t dense_len;
  int64_t index_count;
  int64_t idx_stride;         // elements between consecutive entries of src_idx / dst_idx
  int64_t src_page_rows;      // > 0: paged row addressing of the source side
  int64_t src_page_stride;
  int64_t dst_page_rows;
  int64_t dst_page_stride;
  int32_t plane_inner;        // 1: one grid over (row, plane, piece), planes inside rows
  int32_t dst_major;          // 1: rows are destination rows, their tokens read from the claim tags (plane-major)
};

// Work of one block: kBlockPieces consecutive VEC-byte pieces of the
// flattened (row, piece) range of one plane, two per thread.  The rows the
// range touches (at most kBlockPieces / pieces + 2) are resolved once, into
// LDS, by the block's first threads: source and destination byte offsets, or
// a zero-fill / skip mark.  The copy loop then reads only LDS besides the
// payload, and each thread issues both of its loads before its stores.
constexpr int kBlockPieces = 2 * kBlockThreads;
constexpr int kBlockRows = kBlockPieces + 2;
constexpr int64_t kSkipRow = -1;  // destination offset: the token writes nothing
constexpr int64_t kZeroRow = -1;  // source offset: the destination row is zero filled

// Byte offset of row r inside its plane: r * stride, or for a paged side
// (page_rows > 0) page r / page_rows at page_stride plus row r % page_rows.
__device__ __forceinline__ int64_t row_offset(int64_t r, int64_t page_rows, int64_t page_stride, int64_t stride) {
  if (page_rows <= 0) return r * stride;
  const int64_t pg = r / page_rows;
  return pg * page_stride + (r - pg * page_rows) * stride;
}

// Byte offsets of token u's source and destination rows, with the skip and
// zero-fill marks above.  With DM (destination-major), u is a destination row
// instead: the claim tags (this call's inverse map) name the token that
// writes it, if any.
template <bool DM>
__device__ __forceinline__ void resolve_row(const RowArgs& a, int64_t u, int64_t* so, int64_t* dof) {
  *so = kZeroRow;
  *dof = kSkipRow;
  if constexpr (DM) {
    const uint64_t tag = a.owner[u];
    if (static_cast<uint32_t>(tag >> 32) != a.epoch || static_cast<uint32_t>(tag) == 0u) return;
    const int64_t t = static_cast<int64_t>(static_cast<uint32_t>(tag)) - 1;
    const int64_t srow = a.src_idx ? a.src_idx[t * a.idx_stride] : t + a.src_offset;
    if (srow < 0 || srow >= a.src_rows) return;
    *so = row_offset(srow, a.src_page_rows, a.src_page_stride, a.src_stride);
    *dof = row_offset(u, a.dst_page_rows, a.dst_page_stride, a.dst_stride);
    return;
  }
  int64_t srow = -1;
  int64_t drow = u + a.dst_offset;
  bool valid = false;
  if (u < a.num_tokens) {
    if (a.src_indptr != nullptr) srow = csr_row(a.src_indptr, a.src_idx, a.dense_len, a.index_count, u);
    else srow = a.src_idx ? a.src_idx[u * a.idx_stride] : u + a.src_offset;
    if (a.dst_idx) drow = a.dst_idx[u * a.idx_stride];
    valid = srow >= 0 && srow < a.src_rows && drow >= 0 && drow < a.dst_rows;
    if (valid && a.owner != nullptr) valid = (a.owner[drow] == claim_tag(a.epoch, u));
  }
  if (valid) {
    *so = row_offset(srow, a.src_page_rows, a.src_page_stride, a.src_stride);
    *dof = row_offset(drow, a.dst_page_rows, a.dst_page_stride, a.dst_stride);
  } else if (a.zero_invalid && a.dst_idx == nullptr && drow >= 0 && drow < a.dst_rows) {
    // Only a directly addressed destination row inside its extent is cleared.
    *dof = row_offset(drow, a.dst_page_rows, a.dst_page_stride, a.dst_stride);
  }
}

// INNER = false: plane-major grid (y = plane), rows addressed relative to the
// plane's bases.  INNER = true: one grid over (row, plane) units with absolute
// addresses in LDS and both bases 0; its planes always come from the host
// arrays, whose alignment VEC already covers.  WT (plane-major, 16-byte
// pieces, destination rows of whole 128-byte lines, every destination offset
// below 2 GiB): stores go through a buffer descriptor at the destination
// plane with write-through cache policy (kBufWT; the 1,152-byte MLA rows of
// cfg 5 gather 1.3 % and scatter 0.7 % faster).  Rows that end inside a line
// keep write-back stores: written through, the 656-byte rows of cfg 5 were
// 7 % slower, their shared lines leaving the L2 once per row.
template <int VEC, bool INNER, bool WT = false, bool DM = false>
__global__ __launch_bounds__(kBlockThreads) void row_flat_kernel(const RowArgs a, const int32_t pieces,
                                                                 const float inv_pieces) {
  using V = typename VecType<VEC>::T;
  __shared__ int64_t s_src[kBlockRows];
  __shared__ int64_t s_dst[kBlockRows];
  constexpr bool inner = INNER;
  const int pp = inner ? 0 : a.plane_base + static_cast<int>(blockIdx.y);
  const uint8_t* const sp =
      inner ? nullptr
            : reinterpret_cast<const uint8_t*>(a.src_table ? a.src_table[pp] : a.src_planes[pp - a.plane_base]);
  uint8_t* const dp =
      inner ? nullptr : reinterpret_cast<uint8_t*>(a.dst_table ? a.dst_table[pp] : a.dst_planes[pp - a.plane_base]);
  // Plane bases read from device tables may be less aligned than VEC: such a
  // plane is copied byte by byte (uniform branch).
  const bool narrow = VEC > 1 && ((reinterpret_cast<uintptr_t>(sp) | reinterpret_cast<uintptr_t>(dp)) & (VEC - 1));

  // Block range [l0, l0 + kBlockPieces) starts at piece r0 of unit u0 (a row,
  // or a (row, plane) pair of a plane-inner grid).
  const int64_t l0 = static_cast<int64_t>(blockIdx.x) * kBlockPieces;
  const int64_t u0 = l0 / pieces;
  const int r0 = static_cast<int>(l0 - u0 * pieces);
  const int64_t units = inner ? a.num_rows_out * a.num_planes : a.num_rows_out;
  const int64_t total = units * pieces;
  const int span = static_cast<int>((total - l0) < kBlockPieces ? (total - l0) : kBlockPieces);
  const int nrows = (r0 + span - 1) / pieces + 1;
  for (int i = static_cast<int>(threadIdx.x); i < nrows; i += kBlockThreads) {
    int64_t so, dof;
    if constexpr (!inner) {
      resolve_row<DM>(a, u0 + i, &so, &dof);
    } else {
      const int64_t unit = u0 + i;
      const int64_t row = unit / a.num_planes;
      const int plane = static_cast<int>(unit - row * a.num_planes);
      resolve_row<false>(a, row, &so, &dof);
      if (dof != kSkipRow) dof += static_cast<int64_t>(a.dst_planes[plane]);
      if (so != kZeroRow) so += static_cast<int64_t>(a.src_planes[plane]);
    }
    s_src[i] = so;
    s_dst[i] = dof;
  }
  __syncthreads();

  constexpr int kPer = kBlockPieces / kBlockThreads;
  V v[kPer];
  int64_t d[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int m = static_cast<int>(threadIdx.x) + k * kBlockThreads;  // piece within the block
    d[k] = kSkipRow;
    v[k] = V{};
    if (m >= span) continue;
    // Row and column of piece r0 + m: small integers divided with a float
    // reciprocal and one exact correction step.
    const int q = r0 + m;
    int lt = static_cast<int>(static_cast<float>(q) * inv_pieces);
    if (lt * pieces > q) --lt;
    else if ((lt + 1) * pieces <= q) ++lt;
    const int64_t c = static_cast<int64_t>(q - lt * pieces) * VEC;
    const int64_t dof = s_dst[lt];
    if (dof == kSkipRow) continue;
    d[k] = dof + c;
    const int64_t so = s_src[lt];
    if (so == kZeroRow) continue;
    if (!narrow) {
      v[k] = ldv<VEC>(sp + so + c);
    } else {
#pragma unroll
      for (int b = 0; b < VEC; ++b) dp[d[k] + b] = sp[so + c + b];
      d[k] = kSkipRow;
    }
  }
  if constexpr (WT) {
    static_assert(VEC == 16 && !INNER, "write-through stores take 16-byte pieces of plane-major grids");
    if (!narrow) {
      const buf_t dbuf = make_buf(dp);
#pragma unroll
      for (int k = 0; k < kPer; ++k)
        buf_st16_p<kBufWT>(dbuf, d[k] == kSkipRow ? kOffOob : static_cast<uint32_t>(d[k]), v[k]);
      return;
    }
  }
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    if (d[k] == kSkipRow) continue;
    if (!narrow) {
      stv<VEC>(dp + d[k], v[k]);
    } else {
#pragma unroll
      for (int b = 0; b < VEC; ++b) dp[d[k] + b] = 0;
    }
  }
}

// ----- slot-indexed rows of whole KiB: one wave per KiB, no LDS -----------------------
// The common LMCache / SGLang case: one side addressed by a slot vector, the
// other directly, rows of 1 KiB times a power of two (a 2 KiB bf16 K or V
// token row of 8 heads x 128).  Wave w of a plane moves KiB (w mod units) of
// row w / units: one scalar slot load, then one 16-byte load and store per
// lane through buffer descriptors at the row, masked by offset.  Against the
// block-resolving kernel above, this drops the LDS round trip and barrier and
// needs two rounds of scalar loads before the payload: 10 % off a 256-token
// 2 x NL chunk (67 MB), 2-4 % on batched calls.
struct SlotRowArgs {
  // The fields the first address needs come first (one scalar load).
  const int64_t* idx;          // slots of the indexed side (the source of a gather)
  int64_t num_tokens;          // >= 1
  int32_t units_shift;         // log2(row_bytes / 1024)
  int32_t zero_invalid;        // gather: zero destination rows whose slot is skipped
  int64_t num_rows_out;        // gather: destination rows written (zero tail beyond num_tokens)
  int64_t src_offset;
  int64_t dst_offset;
  int64_t src_rows;
  int64_t dst_rows;
  int64_t src_stride;
  int64_t dst_stride;
  const uint64_t* owner;       // scatter claim tags (nullable)
  uint32_t epoch;
  int32_t pad;
  uint64_t src_planes[kMaxPlanes];
  uint64_t dst_planes[kMaxPlanes];
};

// DM (destination-major scatter): unit u is a destination row, its token read
// from the claim tags (this call's inverse map), so rows are written in
// address order.
template <bool SCATTER, int STP, bool DM = false>
__global__ __launch_bounds__(kBlockThreads) void slot_row_kernel(const SlotRowArgs a) {
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int lane = lane_id();
  const int plane = static_cast<int>(blockIdx.y);
  const int shift = a.units_shift;
  // A gather starts each plane one workgroup (4 KiB) further on.  Destination planes a power of two
  // apart (256-token chunk views of a [2, NL, 4096, 1024] buffer: 8 MiB) otherwise have their
  // resident workgroups write the same offsets of up to 16 planes at once, which made such a chunk
  // 14 % slower (16.3 against 14.3 us); contiguous and other strides are unchanged, the batched
  // gather 1.6 % faster.  Scatters keep the natural order (0.7 % slower rotated).
  const uint32_t bx = SCATTER ? blockIdx.x : (blockIdx.x + blockIdx.y) % gridDim.x;
  const int64_t w = static_cast<int64_t>(bx) * kWavesPerBlock + wave;
  const int64_t u = w >> shift;
  const int64_t part = (w - (u << shift)) << 10;
  const int64_t slot = DM ? static_cast<int64_t>(a.owner[u < a.dst_rows ? u : a.dst_rows - 1])
                          : a.idx[u < a.num_tokens ? u : a.num_tokens - 1];
  const uint64_t sbase = a.src_planes[plane];
  const uint64_t dbase = a.dst_planes[plane];
  // Every argument is read before the first (uniform) branch: one batch of scalar loads.
  asm volatile("" ::"s"(a.num_rows_out), "s"(a.dst_offset), "s"(a.src_offset), "s"(a.src_rows), "s"(a.dst_rows),
               "s"(a.src_stride), "s"(a.dst_stride), "s"(a.zero_invalid), "s"(sbase), "s"(dbase), "s"(slot));
  int64_t srow, drow;
  bool copy, live;
  if constexpr (!SCATTER) {
    srow = u < a.num_tokens ? slot : -1;
    drow = u + a.dst_offset;
    copy = srow >= 0 && srow < a.src_rows;
    live = u < a.num_rows_out && drow >= 0 && drow < a.dst_rows && (copy || a.zero_invalid);
  } else if constexpr (DM) {
    // `slot` holds the tag of destination row u (< dst_rows: the grid covers them).
    const uint64_t tag = static_cast<uint64_t>(slot);
    srow = static_cast<int64_t>(static_cast<uint32_t>(tag)) - 1 + a.src_offset;
    drow = u;
    copy = u < a.dst_rows && static_cast<uint32_t>(tag >> 32) == a.epoch && static_cast<uint32_t>(tag) != 0u &&
           srow >= 0 && srow < a.src_rows;
    live = copy;
  } else {
    srow = u + a.src_offset;
    drow = slot;
    copy = u < a.num_tokens && drow >= 0 && drow < a.dst_rows && srow >= 0 && srow < a.src_rows;
    if (copy && a.owner != nullptr) copy = a.owner[drow] == claim_tag(a.epoch, u);
    live = copy;
  }
  // A skipped side keeps its plane base and an out-of-range offset: the load
  // reads zeros (the zero fill of a skipped gather row), the store is dropped.
  const buf_t sb = make_buf(reinterpret_cast<const uint8_t*>(sbase) + (copy ? srow * a.src_stride + part : 0));
  const buf_t db = make_buf(reinterpret_cast<uint8_t*>(dbase) + (live ? drow * a.dst_stride + part : 0));
  const uint32_t off = static_cast<uint32_t>(lane) * 16u;
  // STP kBufWT (destination rows of whole 128-byte lines): written through
  // the L2, 3 % off a 256-token chunk, 1-2 % on batched calls.
  buf_st16_p<STP>(db, live ? off : kOffOob, buf_ld16(sb, copy ? off : kOffOob));
}

__global__ __launch_bounds__(kBlockThreads) void claim_kernel(const int64_t* idx, int64_t idx_stride,
                                                              const BlockTableSlots bt, const int64_t* src_idx,
                                                              int64_t src_rows, int64_t n, int64_t rows,
                                                              uint64_t* owner, uint32_t epoch, int reset) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // A token whose source is skipped never writes, so it claims nothing.
  if (src_idx != nullptr) {
    const int64_t r = src_idx[i * idx_stride];
    if (r < 0 || r >= src_rows) return;
  }
  const int64_t s = bt.block_tables != nullptr ? block_table_slot(bt, i) : idx[i * idx_stride];
  if (s < 0 || s >= rows) return;
  // The reset pass clears exactly the entries the claim pass will compete for.
  if (reset) {
    owner[s] = 0;
    return;
  }
  atomicMax(reinterpret_cast<unsigned long long*>(owner + s), static_cast<unsigned long long>(claim_tag(epoch, i)));
}

__global__ __launch_bounds__(kBlockThreads) void fill_u64_kernel(uint64_t* p, int64_t n, uint64_t value) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = value;
}

// Largest entry of an int64 vector: workgroup w writes the maximum of the
// entries it visits (grid stride) to partial[w], INT64_MIN if none, and then,
// with a system-scope release, `stamp` to partial[parts + w], so that a host
// thread polling pinned host memory sees the maximum once it sees the stamp.
__global__ __launch_bounds__(kBlockThreads) void index_max_kernel(const int64_t* idx, int64_t n, int64_t* partial,
                                                                  int64_t stamp) {
  int64_t m = INT64_MIN;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    m = idx[i] > m ? idx[i] : m;
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) {
    const int64_t o = __shfl_xor(static_cast<long long>(m), off);
    m = o > m ? o : m;
  }
  __shared__ int64_t wave_max[kWavesPerBlock];
  if (lane_id() == 0) wave_max[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int w = 1; w < kWavesPerBlock; ++w) m = wave_max[w] > m ? wave_max[w] : m;
    partial[blockIdx.x] = m;
    __hip_atomic_store(&partial[gridDim.x + blockIdx.x], stamp, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// ----- strided block transfer ------------------------------------------------------
// Staging [NL, staging_tokens, row_bytes] <-> per-layer pages addressed by block
// id.  Mode 0 pages hold plain rows at block*stride + t*row_bytes; mode 1 pages
// hold all value parts first (t*value_bytes) then all scale parts
// (bs*value_bytes + t*scale_bytes).  Semantics follow the reference kernel text
// csrc/kvcache/kv_transfer_float.mu:3281-3358 (there is no Python reference).
struct StridedArgs {
  uint64_t layers[kMaxPlanes];
  uint8_t* staging;
  const int64_t* block_ids;
  int64_t direction;
  int64_t idx_start;
  int64_t offset_in_object;
  int64_t staging_tokens;
  int64_t block_size;
  int64_t row_bytes;
  int64_t paged_block_stride;
  int64_t mode;
  int64_t value_bytes;
  int64_t scale_bytes;
  int64_t n_valid;
};

template <int VEC>
__global__ __launch_bounds__(kBlockThreads) void strided_block_kernel(const StridedArgs a) {
  const int64_t p = blockIdx.x;
  const int layer = static_cast<int>(blockIdx.y);
  if (p >= a.n_valid) return;
  const int64_t blk = a.block_ids[a.idx_start + p];
  uint8_t* const page = reinterpret_cast<uint8_t*>(a.layers[layer]) + blk * a.paged_block_stride;
  uint8_t* const stage =
      a.staging + ((static_cast<int64_t>(layer) * a.staging_tokens) + a.offset_in_object + p * a.block_size) * a.row_bytes;
  if (a.mode == 0) {
    // Rows of one block are contiguous on both sides.
    const int64_t n = a.block_size * a.row_bytes / VEC;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
      if (a.direction == 0) stv<VEC>(page + i * VEC, ldv<VEC>(stage + i * VEC));
      else stv<VEC>(stage + i * VEC, ldv<VEC>(page + i * VEC));
    }
    return;
  }
  const int64_t row_words = a.row_bytes / VEC;
  const int64_t value_words = a.value_bytes / VEC;
  const int64_t n = a.block_size * row_words;
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) {
    const int64_t t = i / row_words;
    const int64_t w = i - t * row_words;
    uint8_t* const sp = stage + t * a.row_bytes + w * VEC;
    uint8_t* const pp = (w < value_words)
                            ? page + t * a.value_bytes + w * VEC
                            : page + a.block_size * a.value_bytes + t * a.scale_bytes + (w - value_words) * VEC;
    if (a.direction == 0) stv<VEC>(pp, ldv<VEC>(sp));
    else stv<VEC>(sp, ldv<VEC>(pp));
  }
}

// ----- host launchers -----------------------------------------------------------------

namespace {

int vec_for(uint64_t bits) {
  if ((bits & 15u) == 0) return 16;
  if ((bits & 7u) == 0) return 8;
  if ((bits & 3u) == 0) return 4;
  if ((bits & 1u) == 0) return 2;
  return 1;
}

// True when the destination rows of every plane of this launch are whole
// 128-byte lines (row size, strides and host plane bases) and end below 2 GiB
// from their plane base, so 32-bit buffer offsets reach all of them.
bool write_through_rows(const RowArgs& a, int64_t planes) {
  constexpr int64_t kLine = 128;
  if (a.dst_table != nullptr) return false;  // plane bases known only on the device
  if (a.row_bytes % kLine != 0 || a.dst_stride % kLine != 0 || a.dst_page_stride % kLine != 0) return false;
  for (int64_t i = 0; i < planes; ++i)
    if (a.dst_planes[i] % kLine != 0) return false;
  if (a.dst_stride < 0 || a.dst_page_stride < 0 || a.dst_rows <= 0 || a.row_bytes <= 0) return false;
  const __int128 rows = a.dst_rows;
  __int128 end;
  if (a.dst_page_rows > 0)
    end = (rows / a.dst_page_rows + 1) * a.dst_page_stride + static_cast<__int128>(a.dst_page_rows) * a.dst_stride;
  else
    end = rows * a.dst_stride;
  return end + a.row_bytes < (static_cast<__int128>(1) << 31) - 64;
}

// kBlockPieces pieces per block over the flattened (row, piece) range; the
// piece -> row split inside a block stays within small 32-bit integers.
template <int VEC>
hipError_t launch_rows_vec(const RowArgs& a, int64_t planes, hipStream_t stream) {
  const int64_t pieces = a.row_bytes / VEC;
  if (pieces > (int64_t{1} << 22)) return hipErrorInvalidValue;
  const int64_t units = a.plane_inner ? a.num_rows_out * planes : a.num_rows_out;
  const int64_t blocks = (units * pieces + kBlockPieces - 1) / kBlockPieces;
  if (blocks > 0x7FFFFFFF) return hipErrorInvalidValue;
  const dim3 grid(static_cast<uint32_t>(blocks), static_cast<uint32_t>(planes));
  const int32_t np = static_cast<int32_t>(pieces);
  const float inv = 1.0f / static_cast<float>(pieces);
  const bool wt = VEC == 16 && write_through_rows(a, planes);
  if (a.plane_inner)
    hipLaunchKernelGGL((row_flat_kernel<VEC, true>), dim3(static_cast<uint32_t>(blocks)), dim3(kBlockThreads), 0,
                       stream, a, np, inv);
  else if (a.dst_major && wt)
    hipLaunchKernelGGL((row_flat_kernel<16, false, true, true>), grid, dim3(kBlockThreads), 0, stream, a, np, inv);
  else if (a.dst_major)
    hipLaunchKernelGGL((row_flat_kernel<VEC, false, false, true>), grid, dim3(kBlockThreads), 0, stream, a, np, inv);
  else if (wt)
    hipLaunchKernelGGL((row_flat_kernel<16, false, true>), grid, dim3(kBlockThreads), 0, stream, a, np, inv);
  else
    hipLaunchKernelGGL((row_flat_kernel<VEC, false>), grid, dim3(kBlockThreads), 0, stream, a, np, inv);
  return hipGetLastError();
}

}  // namespace

// Scatters whose claim tags are this call's inverse map, with tokens covering
// at least half of the destination rows, run destination-major: rows written
// in address order, sources read wherever they are (random writes cost more
// than random reads on this GPU; each destination row costs one tag read).
// Paged destinations (page-first HiCache tensors, whose rows of one plane sit
// a page stride apart) keep token order: the direct all-layer transfer ran
// 1.42 ms token-major against 1.54 ms destination-major.
bool dst_major(const RowCopyParams& p) {
  return p.owner != nullptr && p.owner_exclusive && p.dst_idx != nullptr && p.idx_stride <= 1 &&
         p.dst_page_rows == 0 && p.num_tokens * 2 >= p.dst_rows && p.dst_rows <= (int64_t{1} << 32);
}

hipError_t launch_row_copy(const RowCopyParams& p, hipStream_t stream) {
  if (p.num_rows_out <= 0 || p.num_planes <= 0 || p.row_bytes <= 0) return hipSuccess;
  if (p.num_rows_out > (int64_t{1} << 32)) return hipErrorInvalidValue;
  if (p.row_bytes > (int64_t{1} << 30)) return hipErrorInvalidValue;
  if (p.src_indptr != nullptr &&
      (p.src_idx == nullptr || p.dense_len <= 0 || p.num_tokens >= (int64_t{1} << 31) || p.dst_idx != nullptr))
    return hipErrorInvalidValue;
  const bool src_host = p.src_table == nullptr;
  const bool dst_host = p.dst_table == nullptr;
  if ((src_host && p.src_planes == nullptr) || (dst_host && p.dst_planes == nullptr)) return hipErrorInvalidValue;

  // Vector width: the largest power of two dividing the row size, both
  // strides and every plane base known on the host.
  if (p.src_page_rows < 0 || p.dst_page_rows < 0) return hipErrorInvalidValue;
  uint64_t bits = static_cast<uint64_t>(p.row_bytes) | static_cast<uint64_t>(p.src_stride) |
                  static_cast<uint64_t>(p.dst_stride);
  if (p.src_page_rows > 0) bits |= static_cast<uint64_t>(p.src_page_stride);
  if (p.dst_page_rows > 0) bits |= static_cast<uint64_t>(p.dst_page_stride);
  for (int64_t i = 0; i < p.num_planes; ++i) {
    if (src_host) bits |= p.src_planes[i];
    if (dst_host) bits |= p.dst_planes[i];
  }
  // Plane bases held in device tables are checked per plane by the kernel.
  const int vec = vec_for(bits);

  // Destination planes closer together than the destination's rows (the
  // layers of one token in a page-first pool): walk planes inside rows, so a
  // token's rows of all planes are written together.  Random reads cost less
  // than random writes on this GPU, so the scattered side moves to the source.
  bool inner = false;
  if (!src_host || !dst_host || p.num_planes < 2 || p.dst_page_rows > 0) {
    inner = false;
  } else {
    uint64_t closest = ~uint64_t{0};
    for (int64_t i = 0; i + 1 < p.num_planes; ++i) {
      const uint64_t gap = p.dst_planes[i + 1] > p.dst_planes[i] ? p.dst_planes[i + 1] - p.dst_planes[i]
                                                                  : p.dst_planes[i] - p.dst_planes[i + 1];
      if (gap < closest) closest = gap;
    }
    inner = p.dst_stride > 0 && closest < static_cast<uint64_t>(p.dst_stride);
  }

  // Slot-indexed rows of 1 KiB x 2^k between host-listed planes: the per-KiB kernel.
  int shift = 0;
  while (shift < 20 && (int64_t{1024} << shift) < p.row_bytes) ++shift;
  const bool one_indexed = (p.src_idx != nullptr) != (p.dst_idx != nullptr);
  if (vec == 16 && (int64_t{1024} << shift) == p.row_bytes && src_host && dst_host && p.src_indptr == nullptr &&
      p.src_page_rows == 0 && p.dst_page_rows == 0 && p.idx_stride <= 1 && !inner && one_indexed &&
      p.num_tokens >= 1) {
    const bool scatter = p.dst_idx != nullptr;
    const bool dm = scatter && dst_major(p);
    const int64_t rows = dm ? p.dst_rows : (scatter ? p.num_tokens : p.num_rows_out);
    const int64_t groups = ((rows << shift) + kWavesPerBlock - 1) / kWavesPerBlock;
    if (rows > (int64_t{1} << 40) || groups > 0x7FFFFFFF) return hipErrorInvalidValue;
    for (int64_t base = 0; base < p.num_planes; base += kMaxPlanes) {
      const int64_t n = (p.num_planes - base) < kMaxPlanes ? (p.num_planes - base) : kMaxPlanes;
      SlotRowArgs a{};
      for (int64_t i = 0; i < n; ++i) {
        a.src_planes[i] = p.src_planes[base + i];
        a.dst_planes[i] = p.dst_planes[base + i];
      }
      a.idx = scatter ? p.dst_idx : p.src_idx;
      a.num_tokens = p.num_tokens;
      a.units_shift = shift;
      a.zero_invalid = p.zero_invalid;
      a.num_rows_out = rows;
      a.src_offset = p.src_offset;
      a.dst_offset = p.dst_offset;
      a.src_rows = p.src_rows;
      a.dst_rows = p.dst_rows;
      a.src_stride = p.src_stride;
      a.dst_stride = p.dst_stride;
      a.owner = p.owner;
      a.epoch = p.epoch;
      const dim3 grid(static_cast<uint32_t>(groups), static_cast<uint32_t>(n));
      bool lines = p.dst_stride % 128 == 0;
      for (int64_t i = 0; i < n; ++i) lines = lines && a.dst_planes[i] % 128 == 0;
      if (dm && lines) hipLaunchKernelGGL((slot_row_kernel<true, kBufWT, true>), grid, dim3(kBlockThreads), 0, stream, a);
      else if (dm) hipLaunchKernelGGL((slot_row_kernel<true, kBufNT, true>), grid, dim3(kBlockThreads), 0, stream, a);
      else if (scatter && lines) hipLaunchKernelGGL((slot_row_kernel<true, kBufWT>), grid, dim3(kBlockThreads), 0, stream, a);
      else if (scatter) hipLaunchKernelGGL((slot_row_kernel<true, kBufNT>), grid, dim3(kBlockThreads), 0, stream, a);
      else if (lines) hipLaunchKernelGGL((slot_row_kernel<false, kBufWT>), grid, dim3(kBlockThreads), 0, stream, a);
      else hipLaunchKernelGGL((slot_row_kernel<false, kBufNT>), grid, dim3(kBlockThreads), 0, stream, a);
      const hipError_t err = hipGetLastError();
      if (err != hipSuccess) return err;
    }
    return hipSuccess;
  }

  for (int64_t base = 0; base < p.num_planes; base += kMaxPlanes) {
    const int64_t n = (p.num_planes - base) < kMaxPlanes ? (p.num_planes - base) : kMaxPlanes;
    RowArgs a{};
    for (int64_t i = 0; i < n; ++i) {
      a.src_planes[i] = src_host ? p.src_planes[base + i] : 0;
      a.dst_planes[i] = dst_host ? p.dst_planes[base + i] : 0;
    }
    a.src_table = p.src_table;
    a.dst_table = p.dst_table;
    a.src_idx = p.src_idx;
    a.dst_idx = p.dst_idx;
    a.owner = p.owner;
    a.num_tokens = p.num_tokens;
    a.num_rows_out = p.num_rows_out;
    a.src_offset = p.src_offset;
    a.dst_offset = p.dst_offset;
    a.src_rows = p.src_rows;
    a.dst_rows = p.dst_rows;
    a.row_bytes = p.row_bytes;
    a.src_stride = p.src_stride;
    a.dst_stride = p.dst_stride;
    a.plane_base = static_cast<int32_t>(base);
    a.num_planes = static_cast<int32_t>(n);
    a.zero_invalid = p.zero_invalid;
    a.epoch = p.epoch;
    a.src_indptr = p.src_indptr;
    a.dense_len = static_cast<uint32_t>(p.dense_len);
    a.index_count = p.index_count;
    a.idx_stride = p.idx_stride > 0 ? p.idx_stride : 1;
    a.src_page_rows = p.src_page_rows;
    a.src_page_stride = p.src_page_stride;
    a.dst_page_rows = p.dst_page_rows;
    a.dst_page_stride = p.dst_page_stride;
    a.plane_inner = inner ? 1 : 0;
    if (!inner && p.src_indptr == nullptr && dst_major(p)) {
      a.dst_major = 1;
      a.num_rows_out = p.dst_rows;
    }
    hipError_t err;
    switch (vec) {
      case 16: err = launch_rows_vec<16>(a, n, stream); break;
      case 8: err = launch_rows_vec<8>(a, n, stream); break;
      case 4: err = launch_rows_vec<4>(a, n, stream); break;
      case 2: err = launch_rows_vec<2>(a, n, stream); break;
      default: err = launch_rows_vec<1>(a, n, stream); break;
    }
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

hipError_t launch_claim(const ClaimSource& src, int64_t n, int64_t rows, uint64_t* owner, uint32_t epoch,
                        hipStream_t stream, bool reset) {
  if (n <= 0) return hipSuccess;
  if ((src.bt.block_tables == nullptr && src.idx == nullptr) || src.idx_stride < 1) return hipErrorInvalidValue;
  const int64_t blocks = (n + kBlockThreads - 1) / kBlockThreads;
  hipLaunchKernelGGL(claim_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kBlockThreads), 0, stream, src.idx,
                     src.idx_stride, src.bt, src.src_idx, src.src_rows, n, rows, owner, epoch, reset ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_index_max(const int64_t* idx, int64_t n, int64_t* partial, int64_t parts, int64_t stamp,
                            hipStream_t stream) {
  if (idx == nullptr || partial == nullptr || n <= 0 || parts < 1 || parts > 4096) return hipErrorInvalidValue;
  hipLaunchKernelGGL(index_max_kernel, dim3(static_cast<uint32_t>(parts)), dim3(kBlockThreads), 0, stream, idx, n,
                     partial, stamp);
  return hipGetLastError();
}

hipError_t launch_fill_u64(uint64_t* p, int64_t n, uint64_t value, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int64_t blocks = (n + kBlockThreads - 1) / kBlockThreads;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(fill_u64_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(kBlockThreads), 0, stream, p, n,
                     value);
  return hipGetLastError();
}

hipError_t launch_strided_blocks(const StridedBlockParams& p, hipStream_t stream) {
  if (p.n_valid <= 0 || p.num_layers <= 0 || p.num_layers > kMaxPlanes || p.block_size <= 0 ||
      p.staging_tokens <= 0 || p.row_bytes <= 0 || (p.row_bytes & 3) != 0 || p.paged_block_stride <= 0)
    return hipErrorInvalidValue;
  if (p.mode != 0 && (p.value_bytes <= 0 || p.scale_bytes <= 0 || (p.value_bytes & 3) != 0 ||
                      (p.scale_bytes & 3) != 0 || p.value_bytes + p.scale_bytes != p.row_bytes))
    return hipErrorInvalidValue;
  if (p.n_valid > 0x7FFFFFFF) return hipErrorInvalidValue;
  StridedArgs a{};
  uint64_t bits = reinterpret_cast<uint64_t>(p.staging) | static_cast<uint64_t>(p.row_bytes) |
                  static_cast<uint64_t>(p.paged_block_stride);
  for (int64_t i = 0; i < p.num_layers; ++i) {
    a.layers[i] = p.paged_ptrs[i];
    bits |= p.paged_ptrs[i];
  }
  if (p.mode != 0) bits |= static_cast<uint64_t>(p.value_bytes) | static_cast<uint64_t>(p.scale_bytes);
  a.staging = p.staging;
  a.block_ids = p.block_ids;
  a.direction = p.direction;
  a.idx_start = p.idx_start;
  a.offset_in_object = p.offset_in_object;
  a.staging_tokens = p.staging_tokens;
  a.block_size = p.block_size;
  a.row_bytes = p.row_bytes;
  a.paged_block_stride = p.paged_block_stride;
  a.mode = p.mode;
  a.value_bytes = p.value_bytes;
  a.scale_bytes = p.scale_bytes;
  a.n_valid = p.n_valid;
  const dim3 grid(static_cast<uint32_t>(p.n_valid), static_cast<uint32_t>(p.num_layers));
  if ((bits & 15u) == 0) hipLaunchKernelGGL(strided_block_kernel<16>, grid, dim3(kBlockThreads), 0, stream, a);
  else hipLaunchKernelGGL(strided_block_kernel<4>, grid, dim3(kBlockThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace kvhip
