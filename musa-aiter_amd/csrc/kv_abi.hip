// C-ABI of libmusa_aiter_kv_hip.so.
//
// The exported names and argument orders are the ones the reference's ctypes
// shims bind (musa_aiter/ops/kv_transfer.py, ops/lmcache_kv_transfer.py), so
// a reference build can load this library in place of its MUSA one.  Every
// entry point returns the HIP status as an int (0 = success); callers that
// bind with restype=None keep working.  The library never synchronises the
// caller's stream except when its duplicate-slot scratch has to grow.
//
// Two generic entry points (musa_aiter_hip_paged_tiles and
// musa_aiter_hip_copy_rows[_table]) carry the strides and flags the Python
// host layer needs (fill_skipped="preserve", merged layouts, non-contiguous
// LMCache buffers, skip prefixes); the reference-named symbols are thin
// wrappers over the same launchers.
#include <atomic>
#include <chrono>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "kv_hip_common.h"
#include "kv_launch.h"
#include "musa_aiter_kv_hip.h"

using kvhip::PagedTileParams;
using kvhip::RowCopyParams;

// Claim tags of musa_aiter_hip_paged_tiles_noalloc: one uint64 per destination
// slot of the caches (16 MiB on every device the library runs on, held until
// the process ends).  In host code `scratch` names a host-side stand-in, not a
// device address: only the per-device address returned by
// hipGetSymbolAddress (noalloc_scratch below) is passed to kernels.
constexpr int64_t kNoAllocMaxSlots = MUSA_AITER_HIP_NOALLOC_MAX_SLOTS;
static __device__ __align__(256) uint64_t scratch[kNoAllocMaxSlots];

namespace {

// ----- duplicate-slot claim scratch --------------------------------------------------------

struct ClaimScratch {
  uint64_t* owner = nullptr;
  int64_t capacity = 0;
  uint32_t epoch = 0;
};

// Eager calls: one array per (device, stream).  Captured calls: one array per
// (device, capture id, capturing stream), so graphs captured one after another
// on the same stream (torch captures every graph on one process-wide stream)
// never share an array, and replays of different graphs may overlap.
using EagerKey = std::pair<int, uintptr_t>;
struct GraphKey {
  int dev;
  unsigned long long capture_id;
  uintptr_t stream;
  bool operator<(const GraphKey& o) const {
    if (dev != o.dev) return dev < o.dev;
    if (capture_id != o.capture_id) return capture_id < o.capture_id;
    return stream < o.stream;
  }
};

std::mutex g_claim_mu;
std::map<EagerKey, ClaimScratch>* g_claims = nullptr;
// Outgrown eager arrays.  Kernels queued before the growth may still read
// them, and freeing would synchronise the device, so they stay allocated;
// capacities double, so they add at most the size of the live arrays.
std::vector<uint64_t*>* g_retired_claims = nullptr;

// Arrays of captured calls.  Each is tied to the graph it was captured into
// by a HIP user object: when the graph (and every executable graph made from
// it) is destroyed, the object's destructor moves the array to a free list
// that later captures on the same device reuse.  g_graph_mu guards only these
// structures and is never held across a HIP call, since the runtime may run
// the destructor from any thread.
struct GraphArray {
  int dev = 0;
  uint64_t* owner = nullptr;
  int64_t capacity = 0;
};
std::mutex g_graph_mu;
std::map<GraphKey, GraphArray>* g_graph_claims = nullptr;  // the live capture's current array, by capture
std::vector<GraphArray>* g_graph_free = nullptr;          // arrays whose graphs were destroyed
int64_t g_graph_arrays = 0;                               // arrays ever allocated for captures

struct GraphRelease {
  GraphKey key;
  GraphArray arr;
};

// User-object destructor (no HIP calls): the graph holding `arr` is gone.
void release_graph_array(void* p) {
  auto* r = static_cast<GraphRelease*>(p);
  {
    std::lock_guard<std::mutex> lock(g_graph_mu);
    auto it = g_graph_claims->find(r->key);
    if (it != g_graph_claims->end() && it->second.owner == r->arr.owner) g_graph_claims->erase(it);
    g_graph_free->push_back(r->arr);
  }
  delete r;
}

// Bytes of device and pinned host memory allocated by the library.
std::atomic<int64_t> g_allocated_bytes{0};

// hipMalloc in relaxed capture mode: another thread's global-mode capture is
// not invalidated, and nothing is recorded into a graph being captured.
hipError_t malloc_relaxed(uint64_t** p, int64_t count) {
  hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
  hipError_t err = hipThreadExchangeStreamCaptureMode(&mode);
  if (err != hipSuccess) return err;
  const size_t bytes = static_cast<size_t>(count) * sizeof(uint64_t);
  const hipError_t merr = hipMalloc(reinterpret_cast<void**>(p), bytes);
  err = hipThreadExchangeStreamCaptureMode(&mode);
  if (merr != hipSuccess) {
    *p = nullptr;
    return merr;
  }
  g_allocated_bytes.fetch_add(static_cast<int64_t>(bytes));
  return err;
}

int64_t grown_capacity(int64_t have, int64_t rows) {
  int64_t cap = have * 2;
  if (cap < rows) cap = rows;
  if (cap < (int64_t{1} << 16)) cap = int64_t{1} << 16;
  return cap;
}

// Claim pass that needs no cleared array: a reset pass zeroes exactly the
// entries the tokens compete for, then the tokens claim with epoch 1.  Used by
// calls captured into graphs (an eager epoch would be frozen into every
// replay, where claims left by earlier replays carry the same epoch and could
// win) and by the allocation-free entry point.
hipError_t reset_and_claim(const kvhip::ClaimSource& src, int64_t n, int64_t rows, uint64_t* owner,
                           hipStream_t stream, const uint64_t** out_owner, uint32_t* epoch) {
  hipError_t err = kvhip::launch_claim(src, n, rows, owner, 1, stream, true);
  if (err != hipSuccess) return err;
  err = kvhip::launch_claim(src, n, rows, owner, 1, stream, false);
  if (err != hipSuccess) return err;
  *out_owner = owner;
  *epoch = 1;
  return hipSuccess;
}

// Claim pass of a call being captured into `graph`: the capture's array (one
// of at least `rows` entries, from the free list or newly allocated and then
// tied to the graph), cleared and claimed by the call itself.
hipError_t prepare_graph_claims(const kvhip::ClaimSource& src, int64_t n, int64_t rows, hipStream_t stream, int dev,
                                unsigned long long capture_id, hipGraph_t graph, const uint64_t** owner,
                                uint32_t* epoch) {
  const GraphKey key{dev, capture_id, reinterpret_cast<uintptr_t>(stream)};
  GraphArray arr;
  bool fresh = false;
  {
    std::lock_guard<std::mutex> lock(g_graph_mu);
    if (g_graph_claims == nullptr) {
      g_graph_claims = new std::map<GraphKey, GraphArray>();
      g_graph_free = new std::vector<GraphArray>();
    }
    auto it = g_graph_claims->find(key);
    if (it != g_graph_claims->end() && it->second.capacity >= rows) {
      arr = it->second;
    } else {
      for (size_t i = 0; i < g_graph_free->size(); ++i) {
        const GraphArray& f = (*g_graph_free)[i];
        if (f.dev == dev && f.capacity >= rows) {
          arr = f;
          (*g_graph_free)[i] = g_graph_free->back();
          g_graph_free->pop_back();
          break;
        }
      }
      fresh = true;
    }
  }
  if (fresh) {
    if (arr.owner == nullptr) {
      arr.dev = dev;
      arr.capacity = grown_capacity(0, rows);
      const hipError_t err = malloc_relaxed(&arr.owner, arr.capacity);
      if (err != hipSuccess) return err;
      std::lock_guard<std::mutex> lock(g_graph_mu);
      ++g_graph_arrays;
    }
    // Tie the array to the graph.  If that fails the array stays with this
    // capture for the life of the process.
    auto* rel = new GraphRelease{key, arr};
    hipUserObject_t obj = nullptr;
    if (hipUserObjectCreate(&obj, rel, release_graph_array, 1, hipUserObjectNoDestructorSync) != hipSuccess) {
      (void)hipGetLastError();
      delete rel;
    } else if (hipGraphRetainUserObject(graph, obj, 1, hipGraphUserObjectMove) != hipSuccess) {
      (void)hipGetLastError();  // the object keeps its reference: the array is never released
    }
    std::lock_guard<std::mutex> lock(g_graph_mu);
    (*g_graph_claims)[key] = arr;
  }
  return reset_and_claim(src, n, rows, arr.owner, stream, owner, epoch);
}

// Runs the claim pass for the `n` destinations of `src` into a destination
// of `rows` rows and returns the tag array and epoch the copy kernel must
// check.  A call that cannot collide (n <= 1) skips the pass.  With caller
// claims (`ws`) the caller's array is used as musa_aiter_hip_claims
// describes.  Otherwise eager calls on one stream share that stream's array
// (stream order keeps them apart), and a captured graph has arrays of its
// own, so one graph must not replay on two streams at once.
//
// *exclusive (optional) tells whether the tags of the returned epoch are
// exactly this call's claims, i.e. the array is the call's inverse map: true
// for epochs no earlier call on the array used, false after a
// reset-and-claim pass.
hipError_t prepare_claims(const kvhip::ClaimSource& src, int64_t n, int64_t rows, hipStream_t stream,
                          const musa_aiter_hip_claims* ws, const uint64_t** owner, uint32_t* epoch,
                          int* exclusive = nullptr) {
  *owner = nullptr;
  *epoch = 0;
  if (exclusive != nullptr) *exclusive = 0;
  if (n <= 1 || rows <= 0 || (src.idx == nullptr && src.bt.block_tables == nullptr)) return hipSuccess;
  if (ws != nullptr) {
    if (ws->tags == nullptr || ws->capacity < rows) return hipErrorInvalidValue;
    if (ws->epoch == 0) return reset_and_claim(src, n, rows, ws->tags, stream, owner, epoch);
    const hipError_t err = kvhip::launch_claim(src, n, rows, ws->tags, ws->epoch, stream);
    if (err != hipSuccess) return err;
    *owner = ws->tags;
    *epoch = ws->epoch;
    if (exclusive != nullptr) *exclusive = 1;
    return hipSuccess;
  }
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  unsigned long long capture_id = 0;
  hipGraph_t graph = nullptr;
  err = hipStreamGetCaptureInfo_v2(stream, &capture, &capture_id, &graph, nullptr, nullptr);
  if (err != hipSuccess) return err;
  if (capture != hipStreamCaptureStatusNone)
    return prepare_graph_claims(src, n, rows, stream, dev, capture_id, graph, owner, epoch);
  std::lock_guard<std::mutex> lock(g_claim_mu);
  if (g_claims == nullptr) g_claims = new std::map<EagerKey, ClaimScratch>();
  ClaimScratch& cs = (*g_claims)[{dev, reinterpret_cast<uintptr_t>(stream)}];
  if (cs.capacity < rows) {
    const int64_t cap = grown_capacity(cs.capacity, rows);
    uint64_t* p = nullptr;
    err = malloc_relaxed(&p, cap);
    if (err != hipSuccess) return err;
    if (cs.owner != nullptr) {
      if (g_retired_claims == nullptr) g_retired_claims = new std::vector<uint64_t*>();
      g_retired_claims->push_back(cs.owner);
    }
    cs.owner = p;
    cs.capacity = cap;
    cs.epoch = 0;
    err = kvhip::launch_fill_u64(cs.owner, cap, 0, stream);
    if (err != hipSuccess) return err;
  }
  if (cs.epoch == 0xFFFFFFFFu) {
    err = kvhip::launch_fill_u64(cs.owner, cs.capacity, 0, stream);
    if (err != hipSuccess) return err;
    cs.epoch = 0;
  }
  cs.epoch += 1;
  err = kvhip::launch_claim(src, n, rows, cs.owner, cs.epoch, stream);
  if (err != hipSuccess) return err;
  *owner = cs.owner;
  *epoch = cs.epoch;
  if (exclusive != nullptr) *exclusive = 1;
  return hipSuccess;
}

// Destinations read from one index vector.
hipError_t prepare_claims(const int64_t* idx, int64_t n, int64_t rows, hipStream_t stream, const uint64_t** owner,
                          uint32_t* epoch, int* exclusive = nullptr) {
  kvhip::ClaimSource src;
  src.idx = idx;
  return prepare_claims(src, n, rows, stream, nullptr, owner, epoch, exclusive);
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Device address of `scratch` on the current device, looked up once per
// device (each device holds its own copy of the array at its own address).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint64_t* g_scratch_ptr[kMaxDevices] = {};

hipError_t noalloc_scratch(uint64_t** out) {
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    // Relaxed capture mode, as for malloc_relaxed: a first call made inside a
    // global-mode capture must not invalidate it.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    err = hipThreadExchangeStreamCaptureMode(&mode);
    if (err != hipSuccess) return err;
    void* ptr = nullptr;
    err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    const hipError_t merr = hipThreadExchangeStreamCaptureMode(&mode);
    if (err == hipSuccess) err = merr;
    if (err != hipSuccess) return err;
    if (ptr == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = static_cast<uint64_t*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

// ----- paged-A helpers -------------------------------------------------------------------

int paged_tiles(int scatter, int codec, int cache_elt, int lin_elt, int lin_dtype, void* kc, void* vc, void* kl,
                void* vl, const int64_t* slots, int64_t nl, int64_t t, int64_t nb, int64_t nh, int64_t hd, int64_t bs,
                int64_t tok_stride_elems, int64_t layer_stride_elems, const float* ks, const float* vs,
                int scale_mode, int fill_zeros, int dedupe, hipStream_t stream,
                const kvhip::BlockTableSlots* bt = nullptr, uint64_t* fixed_owner = nullptr,
                const musa_aiter_hip_claims* ws = nullptr) {
  if (t <= 0 || nl <= 0) return hipSuccess;
  PagedTileParams p{};
  p.scatter = scatter;
  p.codec = codec;
  p.cache_elt = cache_elt;
  p.lin_elt = lin_elt;
  p.lin_dtype = lin_dtype;
  p.cache[0] = kc;
  p.cache[1] = vc;
  p.lin[0] = kl;
  p.lin[1] = vl;
  p.slots = slots;
  p.num_layers = nl;
  p.num_tokens = t;
  p.num_blocks = nb;
  p.num_heads = nh;
  p.head_dim = hd;
  p.block_size = bs;
  p.lin_token_stride = tok_stride_elems * lin_elt;
  p.lin_layer_stride = layer_stride_elems * lin_elt;
  p.scale[0] = ks;
  p.scale[1] = vs;
  p.scale_mode = scale_mode;
  p.fill_zeros = fill_zeros;
  if (bt != nullptr) p.bt = *bt;
  if (scatter && dedupe && t > 1 && t <= kvhip::kScanTokens) {
    // Small scatters find repeated slots inside the kernel (one launch, no
    // tags written; caller-owned tags and the allocation-free entry's array
    // stay untouched, which no later call reads since every call claims under
    // an epoch of its own or clears first); the element kernel cannot, and
    // then the claim pass runs.
    p.scan_dupes = 1;
    const hipError_t err = kvhip::launch_paged_tiles(p, stream);
    if (err != hipErrorNotSupported) return err;
    p.scan_dupes = 0;
  }
  if (scatter && dedupe) {
    kvhip::ClaimSource src;
    src.idx = slots;
    if (bt != nullptr) src.bt = *bt;
    // The allocation-free entry's static array is cleared and claimed per
    // call; otherwise the caller's claims or the library's arrays are used.
    hipError_t err = hipSuccess;
    if (fixed_owner == nullptr) err = prepare_claims(src, t, nb * bs, stream, ws, &p.owner, &p.epoch, &p.owner_exclusive);
    else if (t > 1) err = reset_and_claim(src, t, nb * bs, fixed_owner, stream, &p.owner, &p.epoch);
    if (err != hipSuccess) return err;
  }
  return kvhip::launch_paged_tiles(p, stream);
}

// Paged-A caches <-> dense [batch, dense_len, NH, HD] tensors whose tokens are
// addressed through block tables (the Flash-style preload); the dense side is
// token-major with `tok_stride_elems` elements between tokens.
int dense_tiles(int scatter, int codec, int cache_elt, int lin_elt, int lin_dtype, void* kc, void* vc, void* dk,
                void* dv, const int64_t* block_tables, const int64_t* seq_lens, int64_t batch, int64_t dense_len,
                int64_t max_blocks, int64_t nb, int64_t nh, int64_t hd, int64_t bs, int64_t tok_stride_elems,
                const float* ks, const float* vs, int scale_mode, int fill_zeros, int dedupe,
                const musa_aiter_hip_claims* ws, hipStream_t stream) {
  if (batch <= 0 || dense_len <= 0) return hipSuccess;
  if (block_tables == nullptr || seq_lens == nullptr || max_blocks < 0 || max_blocks >= (int64_t{1} << 31) ||
      dense_len >= (int64_t{1} << 31) || batch >= ((int64_t{1} << 31) - 1) / dense_len + 1)
    return hipErrorInvalidValue;
  kvhip::BlockTableSlots bt{};
  bt.block_tables = block_tables;
  bt.seq_lens = seq_lens;
  bt.num_blocks = nb;
  bt.dense_len = static_cast<uint32_t>(dense_len);
  bt.max_blocks = static_cast<int32_t>(max_blocks);
  bt.block_size = static_cast<int32_t>(bs);
  return paged_tiles(scatter, codec, cache_elt, lin_elt, lin_dtype, kc, vc, dk, dv, nullptr, 1, batch * dense_len,
                     nb, nh, hd, bs, tok_stride_elems, 0, ks, vs, scale_mode, fill_zeros, dedupe, stream, &bt,
                     nullptr, ws);
}

// Dense [batch, dense_len, NH, HD] rows gathered from a token-major cache
// [num_tokens, NH, HD] through a CSR index table; rows without a valid index
// are zeroed.
int csr_dense_rows(const void* kc, const void* vc, const int64_t* indptr, const int64_t* indices, void* ok, void* ov,
                   int64_t batch, int64_t dense_len, int64_t index_count, int64_t num_tokens, int64_t row,
                   hipStream_t stream) {
  if (batch <= 0 || dense_len <= 0 || row <= 0) return hipSuccess;
  if (indptr == nullptr || indices == nullptr || dense_len >= (int64_t{1} << 31) ||
      batch >= ((int64_t{1} << 31) - 1) / dense_len + 1)
    return hipErrorInvalidValue;
  const uint64_t src[2] = {reinterpret_cast<uint64_t>(kc), reinterpret_cast<uint64_t>(vc)};
  const uint64_t dst[2] = {reinterpret_cast<uint64_t>(ok), reinterpret_cast<uint64_t>(ov)};
  RowCopyParams p{};
  p.src_planes = src;
  p.dst_planes = dst;
  p.num_planes = 2;
  p.src_idx = indices;
  p.src_indptr = indptr;
  p.dense_len = dense_len;
  p.index_count = index_count;
  p.num_tokens = batch * dense_len;
  p.num_rows_out = batch * dense_len;
  p.src_rows = num_tokens;
  p.dst_rows = batch * dense_len;
  p.row_bytes = row;
  p.src_stride = row;
  p.dst_stride = row;
  p.zero_invalid = 1;
  return kvhip::launch_row_copy(p, stream);
}

int copy_gather(int elt, void* kc, void* vc, const int64_t* slots, void* ok, void* ov, int64_t nl, int64_t t,
                int64_t nb, int64_t nh, int64_t hd, int64_t bs, int64_t tok_stride, int64_t layer_stride,
                hipStream_t stream) {
  return paged_tiles(0, kvhip::kCopy, elt, elt, kvhip::kLinBF16, kc, vc, ok, ov, slots, nl, t, nb, nh, hd, bs,
                     tok_stride, layer_stride, nullptr, nullptr, 0, 1, 0, stream);
}

int copy_scatter(int elt, const void* kl, const void* vl, const int64_t* slots, void* kc, void* vc, int64_t nl,
                 int64_t t, int64_t nb, int64_t nh, int64_t hd, int64_t bs, int64_t tok_stride, int64_t layer_stride,
                 hipStream_t stream) {
  return paged_tiles(1, kvhip::kCopy, elt, elt, kvhip::kLinBF16, kc, vc, const_cast<void*>(kl),
                     const_cast<void*>(vl), slots, nl, t, nb, nh, hd, bs, tok_stride, layer_stride, nullptr, nullptr,
                     0, 0, 1, stream);
}

// dtype codes of the reference FP8 ABI: 1 = float16, 2 = bfloat16; this
// library also accepts 3 = float32.
bool fp8_lin_dtype(int code, int* lin_dtype, int* lin_elt) {
  switch (code) {
    case 1: *lin_dtype = kvhip::kLinF16; *lin_elt = 2; return true;
    case 2: *lin_dtype = kvhip::kLinBF16; *lin_elt = 2; return true;
    case 3: *lin_dtype = kvhip::kLinF32; *lin_elt = 4; return true;
    default: return false;
  }
}

int fp8_scatter(int codec, const void* kl, const void* vl, const int64_t* slots, void* kc, void* vc, const float* ks,
                const float* vs, int64_t nl, int64_t t, int64_t nb, int64_t nh, int64_t hd, int64_t bs, int dtype_code,
                int scale_mode, hipStream_t stream) {
  int ldt = 0, lelt = 0;
  if (!fp8_lin_dtype(dtype_code, &ldt, &lelt)) return hipErrorInvalidValue;
  return paged_tiles(1, codec, 1, lelt, ldt, kc, vc, const_cast<void*>(kl), const_cast<void*>(vl), slots, nl, t, nb,
                     nh, hd, bs, nh * hd, t * nh * hd, ks, vs, scale_mode, 0, 1, stream);
}

int fp8_gather(int codec, const void* kc, const void* vc, const int64_t* slots, const float* ks, const float* vs,
               void* ok, void* ov, int64_t nl, int64_t t, int64_t nb, int64_t nh, int64_t hd, int64_t bs,
               int dtype_code, int scale_mode, hipStream_t stream) {
  int ldt = 0, lelt = 0;
  if (!fp8_lin_dtype(dtype_code, &ldt, &lelt)) return hipErrorInvalidValue;
  return paged_tiles(0, codec, 1, lelt, ldt, const_cast<void*>(kc), const_cast<void*>(vc), ok, ov, slots, nl, t, nb,
                     nh, hd, bs, nh * hd, t * nh * hd, ks, vs, scale_mode, 1, 0, stream);
}

// ----- row helpers ---------------------------------------------------------------------------

// Gather rows of `planes` slot-addressed caches into directly addressed
// linear rows; rows [num_tokens, rows_out) and skipped tokens are zeroed.
int rows_gather(const uint64_t* cache_planes, const uint64_t* lin_planes, int64_t np, const int64_t* slots,
                int64_t t, int64_t rows_out, int64_t lin_offset, int64_t lin_rows, int64_t slot_rows,
                int64_t row_bytes, int64_t cache_stride, int64_t lin_stride, hipStream_t stream) {
  RowCopyParams p{};
  p.src_planes = cache_planes;
  p.dst_planes = lin_planes;
  p.num_planes = np;
  p.src_idx = slots;
  p.num_tokens = t;
  p.num_rows_out = rows_out;
  p.dst_offset = lin_offset;
  p.src_rows = slot_rows;
  p.dst_rows = lin_rows;
  p.row_bytes = row_bytes;
  p.src_stride = cache_stride;
  p.dst_stride = lin_stride;
  p.zero_invalid = 1;
  return kvhip::launch_row_copy(p, stream);
}

int rows_scatter(const uint64_t* lin_planes, const uint64_t* cache_planes, int64_t np, const int64_t* slots,
                 int64_t t, int64_t lin_offset, int64_t lin_rows, int64_t slot_rows, int64_t row_bytes,
                 int64_t lin_stride, int64_t cache_stride, hipStream_t stream) {
  RowCopyParams p{};
  p.src_planes = lin_planes;
  p.dst_planes = cache_planes;
  p.num_planes = np;
  p.dst_idx = slots;
  p.num_tokens = t;
  p.num_rows_out = t;
  p.src_offset = lin_offset;
  p.src_rows = lin_rows;
  p.dst_rows = slot_rows;
  p.row_bytes = row_bytes;
  p.src_stride = lin_stride;
  p.dst_stride = cache_stride;
  hipError_t err = prepare_claims(slots, t, slot_rows, stream, &p.owner, &p.epoch, &p.owner_exclusive);
  if (err != hipSuccess) return err;
  return kvhip::launch_row_copy(p, stream);
}

uint64_t addr(const void* base, int64_t byte_offset) {
  return reinterpret_cast<uint64_t>(base) + static_cast<uint64_t>(byte_offset);
}

// Whole paged blocks copied between same-layout caches [NL, NB, NH, HD, BS]
// (NL = 1 for single-layer caches): `mapping` holds [num_pairs, 2] (source,
// destination) block ids.  A pair with a negative or out-of-range id is
// skipped; a destination named by several pairs keeps the last one.  One
// block of one plane is one row of nh * hd * bs * elt bytes.
int copy_blocks(int64_t elt, const void* sk, const void* sv, void* dk, void* dv, const int64_t* mapping,
                int64_t num_pairs, int64_t nl, int64_t src_blocks, int64_t dst_blocks, int64_t nh, int64_t hd,
                int64_t bs, hipStream_t stream, const musa_aiter_hip_claims* ws = nullptr) {
  if (num_pairs <= 0 || nl <= 0) return hipSuccess;
  if (mapping == nullptr || nh <= 0 || hd <= 0 || bs <= 0 || src_blocks < 0 || dst_blocks < 0)
    return hipErrorInvalidValue;
  const int64_t row = nh * hd * bs * elt;
  std::vector<uint64_t> src, dst;
  for (int64_t kv = 0; kv < 2; ++kv)
    for (int64_t l = 0; l < nl; ++l) {
      src.push_back(addr(kv == 0 ? sk : sv, l * src_blocks * row));
      dst.push_back(addr(kv == 0 ? dk : dv, l * dst_blocks * row));
    }
  RowCopyParams p{};
  p.src_planes = src.data();
  p.dst_planes = dst.data();
  p.num_planes = 2 * nl;
  p.src_idx = mapping;
  p.dst_idx = mapping + 1;
  p.idx_stride = 2;
  p.num_tokens = num_pairs;
  p.num_rows_out = num_pairs;
  p.src_rows = src_blocks;
  p.dst_rows = dst_blocks;
  p.row_bytes = row;
  p.src_stride = row;
  p.dst_stride = row;
  kvhip::ClaimSource claims;
  claims.idx = mapping + 1;
  claims.idx_stride = 2;
  claims.src_idx = mapping;
  claims.src_rows = src_blocks;
  hipError_t err = prepare_claims(claims, num_pairs, dst_blocks, stream, ws, &p.owner, &p.epoch, &p.owner_exclusive);
  if (err != hipSuccess) return err;
  return kvhip::launch_row_copy(p, stream);
}

// LMCache legacy 6-D cache [NL, 2, NB, BS, NH, HS] <-> buffer [2, NL, T, NH*HS].
int lmcache_6d(int scatter, int elt, const void* buffer, const void* paged, const int64_t* slots, int64_t nl,
               int64_t t, int64_t nb, int64_t bs, int64_t nh, int64_t hs, hipStream_t stream) {
  if (nl <= 0 || t <= 0) return hipSuccess;
  const int64_t row = nh * hs * elt;
  std::vector<uint64_t> cache_planes, lin_planes;
  for (int64_t kv = 0; kv < 2; ++kv)
    for (int64_t l = 0; l < nl; ++l) {
      cache_planes.push_back(addr(paged, ((l * 2 + kv) * nb * bs) * row));
      lin_planes.push_back(addr(buffer, (kv * nl + l) * t * row));
    }
  if (scatter)
    return rows_scatter(lin_planes.data(), cache_planes.data(), 2 * nl, slots, t, 0, t, nb * bs, row, row, row,
                        stream);
  return rows_gather(cache_planes.data(), lin_planes.data(), 2 * nl, slots, t, t, 0, t, nb * bs, row, row, row,
                     stream);
}

// LMCache MLA [NL, NB, BS, D] <-> [NL, T, D].
int lmcache_mla(int scatter, int elt, const void* buffer, const void* paged, const int64_t* slots, int64_t nl,
                int64_t t, int64_t nb, int64_t bs, int64_t d, hipStream_t stream) {
  if (nl <= 0 || t <= 0) return hipSuccess;
  const int64_t row = d * elt;
  std::vector<uint64_t> cache_planes, lin_planes;
  for (int64_t l = 0; l < nl; ++l) {
    cache_planes.push_back(addr(paged, l * nb * bs * row));
    lin_planes.push_back(addr(buffer, l * t * row));
  }
  if (scatter)
    return rows_scatter(lin_planes.data(), cache_planes.data(), nl, slots, t, 0, t, nb * bs, row, row, row, stream);
  return rows_gather(cache_planes.data(), lin_planes.data(), nl, slots, t, t, 0, t, nb * bs, row, row, row, stream);
}

// Split K/V planes of one layer for 2xNL / list layouts: buffer [2, NL, M, H].
int lmcache_planes(int scatter, int elt, const void* memory, const uint64_t* cache_planes, const int64_t* axes,
                   const int64_t* layers, int64_t np, const int64_t* slots, int64_t nl, int64_t m, int64_t t,
                   int64_t skip, int64_t nb, int64_t bs, int64_t hidden, int zero_tail, hipStream_t stream) {
  if (t <= 0 || np <= 0) return hipSuccess;
  const int64_t row = hidden * elt;
  std::vector<uint64_t> lin_planes(np);
  for (int64_t i = 0; i < np; ++i) lin_planes[i] = addr(memory, (axes[i] * nl + layers[i]) * m * row);
  if (scatter)
    return rows_scatter(lin_planes.data(), cache_planes, np, slots, t, skip, m, nb * bs, row, row, row, stream);
  const int64_t rows_out = zero_tail ? (m - skip) : t;
  return rows_gather(cache_planes, lin_planes.data(), np, slots, t, rows_out, skip, m, nb * bs, row, row, row, stream);
}

}  // namespace

extern "C" {

// ----- identity / ABI probes ----------------------------------------------------------------

int musa_aiter_kv_transfer_abi_version() { return 1; }
int native_lmcache_kv_transfer_abi_version() { return 1; }
int musa_aiter_fp8_kv_cache_abi_version() { return 1; }
int musa_aiter_dsv4_kv_copy_abi_version() { return 1; }
const char* musa_aiter_hip_backend_name() { return "rocm-hip"; }
const char* musa_aiter_hip_error_string(int code) { return hipGetErrorString(static_cast<hipError_t>(code)); }

int musa_aiter_hip_block_pattern_copy(const void* src, void* dst, const int32_t* src_blocks,
                                      const int32_t* dst_blocks, int64_t num_blocks, int64_t src_region_blocks,
                                      int64_t dst_region_blocks, int64_t src_block_bytes, int64_t dst_block_bytes,
                                      int64_t planes, int64_t src_plane_stride, int64_t dst_plane_stride,
                                      int write_through, void* stream) {
  kvhip::BlockPatternParams p{};
  p.src = src;
  p.dst = dst;
  p.src_blocks = src_blocks;
  p.dst_blocks = dst_blocks;
  p.num_blocks = num_blocks;
  p.src_region_blocks = src_region_blocks;
  p.dst_region_blocks = dst_region_blocks;
  p.src_block_bytes = src_block_bytes;
  p.dst_block_bytes = dst_block_bytes;
  p.planes = planes;
  p.src_plane_stride = src_plane_stride;
  p.dst_plane_stride = dst_plane_stride;
  p.write_through = write_through != 0;
  return kvhip::launch_block_pattern(p, as_stream(stream));
}

int64_t musa_aiter_hip_graph_claim_arrays() {
  std::lock_guard<std::mutex> lock(g_graph_mu);
  return g_graph_arrays;
}

int64_t musa_aiter_hip_allocated_bytes() { return g_allocated_bytes.load(); }

int musa_aiter_hip_index_max(const int64_t* idx, int64_t n, int64_t* partial, int64_t parts, int64_t stamp,
                             void* stream) {
  if (stamp == 0) return hipErrorInvalidValue;
  hipError_t err = kvhip::launch_index_max(idx, n, partial, parts, stamp, as_stream(stream));
  if (err != hipSuccess) return err;
  // The stamps arrive as the kernel ends; polling them returns sooner than a
  // stream synchronisation.  A kernel that has not run after 0.2 s (the
  // stream busy with earlier work) is waited for by the synchronisation.
  const auto deadline = std::chrono::steady_clock::now() + std::chrono::milliseconds(200);
  for (int64_t w = 0; w < parts;) {
    if (__atomic_load_n(&partial[parts + w], __ATOMIC_ACQUIRE) == stamp) {
      ++w;
    } else if (std::chrono::steady_clock::now() > deadline) {
      return hipStreamSynchronize(as_stream(stream));
    } else {
      __builtin_ia32_pause();
    }
  }
  return hipSuccess;
}

// ----- generic entries used by the Python host layer ----------------------------------------

int musa_aiter_hip_paged_tiles(int scatter, int codec, int cache_elt, int lin_elt, int lin_dtype, void* key_cache,
                               void* value_cache, void* key_linear, void* value_linear, const int64_t* slot_mapping,
                               int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,
                               int64_t head_dim, int64_t block_size, int64_t lin_token_stride,
                               int64_t lin_layer_stride, const float* k_scale, const float* v_scale, int scale_mode,
                               int fill_zeros, int dedupe, const musa_aiter_hip_claims* claims, void* stream) {
  return paged_tiles(scatter, codec, cache_elt, lin_elt, lin_dtype, key_cache, value_cache, key_linear, value_linear,
                     slot_mapping, num_layers, num_tokens, num_blocks, num_heads, head_dim, block_size,
                     lin_token_stride, lin_layer_stride, k_scale, v_scale, scale_mode, fill_zeros, dedupe,
                     as_stream(stream), nullptr, nullptr, claims);
}

int musa_aiter_hip_paged_tiles_noalloc(int scatter, int codec, int cache_elt, int lin_elt, int lin_dtype,
                                       void* key_cache, void* value_cache, void* key_linear, void* value_linear,
                                       const int64_t* slot_mapping, int64_t num_layers, int64_t num_tokens,
                                       int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size,
                                       int64_t lin_token_stride, int64_t lin_layer_stride, const float* k_scale,
                                       const float* v_scale, int scale_mode, int fill_zeros, int dedupe,
                                       void* stream) {
  uint64_t* owner = nullptr;
  if (scatter && dedupe) {
    if (num_blocks < 0 || block_size <= 0 || num_blocks > kNoAllocMaxSlots / block_size) return hipErrorInvalidValue;
    const hipError_t err = noalloc_scratch(&owner);
    if (err != hipSuccess) return err;
  }
  return paged_tiles(scatter, codec, cache_elt, lin_elt, lin_dtype, key_cache, value_cache, key_linear, value_linear,
                     slot_mapping, num_layers, num_tokens, num_blocks, num_heads, head_dim, block_size,
                     lin_token_stride, lin_layer_stride, k_scale, v_scale, scale_mode, fill_zeros, dedupe,
                     as_stream(stream), nullptr, owner);
}

int musa_aiter_hip_paged_dense_tiles(int scatter, int codec, int cache_elt, int lin_elt, int lin_dtype,
                                     void* key_cache, void* value_cache, void* dense_k, void* dense_v,
                                     const int64_t* block_tables, const int64_t* seq_lens, int64_t batch,
                                     int64_t dense_len, int64_t max_blocks, int64_t num_blocks, int64_t num_heads,
                                     int64_t head_dim, int64_t block_size, int64_t dense_token_stride,
                                     const float* k_scale, const float* v_scale, int scale_mode, int fill_zeros,
                                     int dedupe, const musa_aiter_hip_claims* claims, void* stream) {
  return dense_tiles(scatter, codec, cache_elt, lin_elt, lin_dtype, key_cache, value_cache, dense_k, dense_v,
                     block_tables, seq_lens, batch, dense_len, max_blocks, num_blocks, num_heads, head_dim,
                     block_size, dense_token_stride, k_scale, v_scale, scale_mode, fill_zeros, dedupe, claims,
                     as_stream(stream));
}

int musa_aiter_hip_csr_dense_rows(const void* key_cache, const void* value_cache, const int64_t* kv_indptr,
                                  const int64_t* kv_indices, void* out_k, void* out_v, int64_t batch,
                                  int64_t dense_len, int64_t index_count, int64_t num_tokens, int64_t row_bytes,
                                  void* stream) {
  return csr_dense_rows(key_cache, value_cache, kv_indptr, kv_indices, out_k, out_v, batch, dense_len, index_count,
                        num_tokens, row_bytes, as_stream(stream));
}

int musa_aiter_hip_copy_rows(const uint64_t* src_planes, const uint64_t* dst_planes, const uint64_t* src_table,
                             const uint64_t* dst_table, int64_t num_planes, const int64_t* src_idx,
                             const int64_t* dst_idx, int64_t num_tokens, int64_t num_rows_out, int64_t src_offset,
                             int64_t dst_offset, int64_t src_rows, int64_t dst_rows, int64_t row_bytes,
                             int64_t src_stride, int64_t dst_stride, int zero_invalid, int dedupe,
                             const musa_aiter_hip_claims* claims, void* stream) {
  RowCopyParams p{};
  p.src_planes = src_planes;
  p.dst_planes = dst_planes;
  p.src_table = src_table;
  p.dst_table = dst_table;
  p.num_planes = num_planes;
  p.src_idx = src_idx;
  p.dst_idx = dst_idx;
  p.num_tokens = num_tokens;
  p.num_rows_out = num_rows_out;
  p.src_offset = src_offset;
  p.dst_offset = dst_offset;
  p.src_rows = src_rows;
  p.dst_rows = dst_rows;
  p.row_bytes = row_bytes;
  p.src_stride = src_stride;
  p.dst_stride = dst_stride;
  p.zero_invalid = zero_invalid;
  if (dedupe && dst_idx != nullptr) {
    kvhip::ClaimSource src;
    src.idx = dst_idx;
    src.src_idx = src_idx;
    src.src_rows = src_rows;
    hipError_t err =
        prepare_claims(src, num_tokens, dst_rows, as_stream(stream), claims, &p.owner, &p.epoch, &p.owner_exclusive);
    if (err != hipSuccess) return err;
  }
  return kvhip::launch_row_copy(p, as_stream(stream));
}

static_assert(sizeof(musa_aiter_hip_copy_rows_call) == 144, "the Python host layer packs 144 bytes");

int musa_aiter_hip_copy_rows_packed(const musa_aiter_hip_copy_rows_call* call, void* stream) {
  if (call == nullptr) return hipErrorInvalidValue;
  musa_aiter_hip_copy_rows_call c;
  std::memcpy(&c, call, sizeof c);  // the caller's buffer need not be aligned
  return musa_aiter_hip_copy_rows(c.src_planes, c.dst_planes, c.src_table, c.dst_table, c.num_planes, c.src_idx,
                                  c.dst_idx, c.num_tokens, c.num_rows_out, c.src_offset, c.dst_offset, c.src_rows,
                                  c.dst_rows, c.row_bytes, c.src_stride, c.dst_stride, c.zero_invalid, c.dedupe,
                                  c.claims, stream);
}

// ----- paged-A copies (kv_transfer.py:350-376, :410-436, :480-508, :542-570) ----------------

#define KVHIP_PAGED_COPY(SUFFIX, ELT)                                                                              \
  int musa_aiter_kv_paged_to_linear_##SUFFIX(const void* key_cache, const void* value_cache,                      \
                                             const int64_t* slot_mapping, void* out_k, void* out_v,               \
                                             int64_t num_tokens, int64_t num_blocks, int64_t num_heads,           \
                                             int64_t head_dim, int64_t block_size, void* stream) {                \
    return copy_gather(ELT, const_cast<void*>(key_cache), const_cast<void*>(value_cache), slot_mapping, out_k,    \
                       out_v, 1, num_tokens, num_blocks, num_heads, head_dim, block_size, num_heads * head_dim, 0, \
                       as_stream(stream));                                                                        \
  }                                                                                                               \
  int musa_aiter_kv_linear_to_paged_##SUFFIX(const void* key_linear, const void* value_linear,                    \
                                             const int64_t* slot_mapping, void* key_cache, void* value_cache,     \
                                             int64_t num_tokens, int64_t num_blocks, int64_t num_heads,           \
                                             int64_t head_dim, int64_t block_size, void* stream) {                \
    return copy_scatter(ELT, key_linear, value_linear, slot_mapping, key_cache, value_cache, 1, num_tokens,       \
                        num_blocks, num_heads, head_dim, block_size, num_heads * head_dim, 0, as_stream(stream)); \
  }                                                                                                               \
  int musa_aiter_kv_paged_to_linear_multi_layer_##SUFFIX(                                                         \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, void* out_k, void* out_v,      \
      int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t num_heads, int64_t head_dim,            \
      int64_t block_size, void* stream) {                                                                         \
    return copy_gather(ELT, const_cast<void*>(key_cache), const_cast<void*>(value_cache), slot_mapping, out_k,    \
                       out_v, num_layers, num_tokens, num_blocks, num_heads, head_dim, block_size,                \
                       num_heads * head_dim, num_tokens * num_heads * head_dim, as_stream(stream));               \
  }                                                                                                               \
  int musa_aiter_kv_linear_to_paged_multi_layer_##SUFFIX(                                                         \
      const void* key_linear, const void* value_linear, const int64_t* slot_mapping, void* key_cache,             \
      void* value_cache, int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,           \
      int64_t head_dim, int64_t block_size, void* stream) {                                                       \
    return copy_scatter(ELT, key_linear, value_linear, slot_mapping, key_cache, value_cache, num_layers,          \
                        num_tokens, num_blocks, num_heads, head_dim, block_size, num_heads * head_dim,            \
                        num_tokens * num_heads * head_dim, as_stream(stream));                                    \
  }                                                                                                               \
  int musa_aiter_kv_paged_to_merged_linear_##SUFFIX(const void* key_cache, const void* value_cache,               \
                                                    const int64_t* slot_mapping, void* out, int64_t num_tokens,   \
                                                    int64_t num_blocks, int64_t num_heads, int64_t head_dim,      \
                                                    int64_t block_size, void* stream) {                           \
    const int64_t row = num_heads * head_dim;                                                                     \
    return copy_gather(ELT, const_cast<void*>(key_cache), const_cast<void*>(value_cache), slot_mapping, out,      \
                       static_cast<uint8_t*>(out) + row * ELT, 1, num_tokens, num_blocks, num_heads, head_dim,    \
                       block_size, 2 * row, 0, as_stream(stream));                                                \
  }                                                                                                               \
  int musa_aiter_kv_merged_linear_to_paged_##SUFFIX(const void* merged, const int64_t* slot_mapping,              \
                                                    void* key_cache, void* value_cache, int64_t num_tokens,       \
                                                    int64_t num_blocks, int64_t num_heads, int64_t head_dim,      \
                                                    int64_t block_size, void* stream) {                           \
    const int64_t row = num_heads * head_dim;                                                                     \
    return copy_scatter(ELT, merged, static_cast<const uint8_t*>(merged) + row * ELT, slot_mapping, key_cache,    \
                        value_cache, 1, num_tokens, num_blocks, num_heads, head_dim, block_size, 2 * row, 0,      \
                        as_stream(stream));                                                                       \
  }                                                                                                               \
  int musa_aiter_kv_paged_to_merged_linear_multi_layer_##SUFFIX(                                                  \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, void* out, int64_t num_layers, \
      int64_t num_tokens, int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size,            \
      void* stream) {                                                                                             \
    const int64_t row = num_heads * head_dim;                                                                     \
    return copy_gather(ELT, const_cast<void*>(key_cache), const_cast<void*>(value_cache), slot_mapping, out,      \
                       static_cast<uint8_t*>(out) + row * ELT, num_layers, num_tokens, num_blocks, num_heads,     \
                       head_dim, block_size, 2 * row, 2 * row * num_tokens, as_stream(stream));                   \
  }                                                                                                               \
  int musa_aiter_kv_merged_linear_to_paged_multi_layer_##SUFFIX(                                                  \
      const void* merged, const int64_t* slot_mapping, void* key_cache, void* value_cache, int64_t num_layers,    \
      int64_t num_tokens, int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size,            \
      void* stream) {                                                                                             \
    const int64_t row = num_heads * head_dim;                                                                     \
    return copy_scatter(ELT, merged, static_cast<const uint8_t*>(merged) + row * ELT, slot_mapping, key_cache,    \
                        value_cache, num_layers, num_tokens, num_blocks, num_heads, head_dim, block_size,         \
                        2 * row, 2 * row * num_tokens, as_stream(stream));                                        \
  }                                                                                                               \
  int musa_aiter_kv_paged_to_mla_linear_##SUFFIX(const void* kv_cache, const void* pe_cache,                     \
                                                 const int64_t* slot_mapping, void* out_kv, void* out_pe,         \
                                                 int64_t num_tokens, int64_t num_blocks, int64_t block_size,      \
                                                 int64_t kv_dim, int64_t pe_dim, void* stream) {                  \
    const uint64_t kc = addr(kv_cache, 0), pc = addr(pe_cache, 0), ko = addr(out_kv, 0), po = addr(out_pe, 0);   \
    const int64_t slots = num_blocks * block_size;                                                                \
    int err = rows_gather(&kc, &ko, 1, slot_mapping, num_tokens, num_tokens, 0, num_tokens, slots, kv_dim * ELT,  \
                          kv_dim * ELT, kv_dim * ELT, as_stream(stream));                                         \
    if (err != 0) return err;                                                                                     \
    return rows_gather(&pc, &po, 1, slot_mapping, num_tokens, num_tokens, 0, num_tokens, slots, pe_dim * ELT,     \
                       pe_dim * ELT, pe_dim * ELT, as_stream(stream));                                            \
  }                                                                                                               \
  int musa_aiter_kv_mla_linear_to_paged_##SUFFIX(const void* kv_linear, const void* pe_linear,                   \
                                                 const int64_t* slot_mapping, void* kv_cache, void* pe_cache,     \
                                                 int64_t num_tokens, int64_t num_blocks, int64_t block_size,      \
                                                 int64_t kv_dim, int64_t pe_dim, void* stream) {                  \
    const uint64_t src[2] = {addr(kv_linear, 0), addr(pe_linear, 0)};                                             \
    const uint64_t dst[2] = {addr(kv_cache, 0), addr(pe_cache, 0)};                                               \
    const int64_t slots = num_blocks * block_size;                                                                \
    RowCopyParams p{};                                                                                            \
    p.num_planes = 1;                                                                                             \
    p.dst_idx = slot_mapping;                                                                                     \
    p.num_tokens = num_tokens;                                                                                    \
    p.num_rows_out = num_tokens;                                                                                  \
    p.src_rows = num_tokens;                                                                                      \
    p.dst_rows = slots;                                                                                           \
    int err = prepare_claims(slot_mapping, num_tokens, slots, as_stream(stream), &p.owner, &p.epoch,              \
                             &p.owner_exclusive);                                                                 \
    if (err != 0) return err;                                                                                     \
    const int64_t dims[2] = {kv_dim, pe_dim};                                                                     \
    for (int i = 0; i < 2; ++i) {                                                                                 \
      p.src_planes = &src[i];                                                                                     \
      p.dst_planes = &dst[i];                                                                                     \
      p.row_bytes = dims[i] * ELT;                                                                                \
      p.src_stride = dims[i] * ELT;                                                                               \
      p.dst_stride = dims[i] * ELT;                                                                               \
      err = kvhip::launch_row_copy(p, as_stream(stream));                                                         \
      if (err != 0) return err;                                                                                   \
    }                                                                                                             \
    return 0;                                                                                                     \
  }

KVHIP_PAGED_COPY(float, 4)
KVHIP_PAGED_COPY(half, 2)
KVHIP_PAGED_COPY(bfloat16, 2)
#undef KVHIP_PAGED_COPY

// ----- dense preload (kv_transfer.py:1220-1288, :1369-1440, :1443-1524) -----------------------

#define KVHIP_DENSE(SUFFIX, ELT)                                                                                   \
  int musa_aiter_kv_load_and_reshape_flash_##SUFFIX(                                                              \
      const void* key_cache, const void* value_cache, const int64_t* block_tables, const int64_t* seq_lens,       \
      void* out_k, void* out_v, int64_t batch, int64_t dense_len, int64_t max_blocks, int64_t num_blocks,         \
      int64_t num_heads, int64_t head_dim, int64_t block_size, void* stream) {                                    \
    return dense_tiles(0, kvhip::kCopy, ELT, ELT, kvhip::kLinBF16, const_cast<void*>(key_cache),                  \
                       const_cast<void*>(value_cache), out_k, out_v, block_tables, seq_lens, batch, dense_len,    \
                       max_blocks, num_blocks, num_heads, head_dim, block_size, num_heads * head_dim, nullptr,    \
                       nullptr, 0, 1, 0, nullptr, as_stream(stream));                                            \
  }                                                                                                               \
  int musa_aiter_kv_reshape_and_cache_back_flash_##SUFFIX(                                                        \
      const void* dense_k, const void* dense_v, const int64_t* block_tables, const int64_t* seq_lens,             \
      void* key_cache, void* value_cache, int64_t batch, int64_t dense_len, int64_t max_blocks,                   \
      int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size, void* stream) {                \
    return dense_tiles(1, kvhip::kCopy, ELT, ELT, kvhip::kLinBF16, key_cache, value_cache,                        \
                       const_cast<void*>(dense_k), const_cast<void*>(dense_v), block_tables, seq_lens, batch,     \
                       dense_len, max_blocks, num_blocks, num_heads, head_dim, block_size, num_heads * head_dim,  \
                       nullptr, nullptr, 0, 0, 1, nullptr, as_stream(stream));                                   \
  }                                                                                                               \
  int musa_aiter_kv_triton_indexed_to_dense_##SUFFIX(                                                             \
      const void* key_cache, const void* value_cache, const int64_t* kv_indptr, const int64_t* kv_indices,        \
      void* out_k, void* out_v, int64_t batch, int64_t dense_len, int64_t index_count, int64_t num_tokens,        \
      int64_t num_heads, int64_t head_dim, void* stream) {                                                        \
    if (num_heads <= 0 || head_dim <= 0) return hipSuccess;                                                       \
    return csr_dense_rows(key_cache, value_cache, kv_indptr, kv_indices, out_k, out_v, batch, dense_len,          \
                          index_count, num_tokens, num_heads * head_dim * ELT, as_stream(stream));               \
  }

KVHIP_DENSE(float, 4)
KVHIP_DENSE(half, 2)
KVHIP_DENSE(bfloat16, 2)
#undef KVHIP_DENSE

// ----- paged block copies (kv_transfer.py:1798-1868 FP8, :1962-2032) ---------------------------

#define KVHIP_BLOCKS(NAME, ELT)                                                                                    \
  int NAME(const void* src_key_cache, const void* src_value_cache, void* dst_key_cache, void* dst_value_cache,    \
           const int64_t* block_mapping, int64_t num_pairs, int64_t num_layers, int64_t src_blocks,               \
           int64_t dst_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size, void* stream) {           \
    return copy_blocks(ELT, src_key_cache, src_value_cache, dst_key_cache, dst_value_cache, block_mapping,        \
                       num_pairs, num_layers, src_blocks, dst_blocks, num_heads, head_dim, block_size,            \
                       as_stream(stream));                                                                        \
  }

KVHIP_BLOCKS(musa_aiter_kv_copy_paged_blocks_float, 4)
KVHIP_BLOCKS(musa_aiter_kv_copy_paged_blocks_half, 2)
KVHIP_BLOCKS(musa_aiter_kv_copy_paged_blocks_bfloat16, 2)
KVHIP_BLOCKS(musa_aiter_kv_copy_paged_blocks_fp8_vec8, 1)
#undef KVHIP_BLOCKS

int musa_aiter_hip_copy_blocks(const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                               const int64_t* block_mapping, int64_t num_pairs, int64_t num_layers,
                               int64_t src_blocks, int64_t dst_blocks, int64_t block_bytes,
                               const musa_aiter_hip_claims* claims, void* stream) {
  return copy_blocks(1, src_k, src_v, dst_k, dst_v, block_mapping, num_pairs, num_layers, src_blocks, dst_blocks, 1,
                     block_bytes, 1, as_stream(stream), claims);
}

// ----- FP8 quant-store / dequant-gather (kv_transfer.py:2446-2480 and the other FP8 shims) -----

#define KVHIP_FP8(FMT, CODEC)                                                                                      \
  int musa_aiter_kv_linear_to_paged_fp8_##FMT(const void* key_linear, const void* value_linear,                   \
                                              const int64_t* slot_mapping, void* key_cache, void* value_cache,    \
                                              const float* k_scale, const float* v_scale, int64_t num_tokens,     \
                                              int64_t num_blocks, int64_t num_heads, int64_t head_dim,            \
                                              int64_t block_size, int dtype_code, void* stream) {                 \
    return fp8_scatter(CODEC, key_linear, value_linear, slot_mapping, key_cache, value_cache, k_scale, v_scale,   \
                       1, num_tokens, num_blocks, num_heads, head_dim, block_size, dtype_code, 0,                 \
                       as_stream(stream));                                                                        \
  }                                                                                                               \
  int musa_aiter_kv_linear_to_paged_fp8_vec4_##FMT(                                                               \
      const void* key_linear, const void* value_linear, const int64_t* slot_mapping, void* key_cache,             \
      void* value_cache, const float* k_scale, const float* v_scale, int64_t num_tokens, int64_t num_blocks,      \
      int64_t num_heads, int64_t head_dim, int64_t block_size, int dtype_code, void* stream, int scale_mode) {    \
    return fp8_scatter(CODEC, key_linear, value_linear, slot_mapping, key_cache, value_cache, k_scale, v_scale,   \
                       1, num_tokens, num_blocks, num_heads, head_dim, block_size, dtype_code, scale_mode,        \
                       as_stream(stream));                                                                        \
  }                                                                                                               \
  int musa_aiter_kv_paged_fp8_to_linear_##FMT(const void* key_cache, const void* value_cache,                     \
                                              const int64_t* slot_mapping, const float* k_scale,                  \
                                              const float* v_scale, void* out_k, void* out_v, int64_t num_tokens, \
                                              int64_t num_blocks, int64_t num_heads, int64_t head_dim,            \
                                              int64_t block_size, int dtype_code, void* stream) {                 \
    return fp8_gather(CODEC, key_cache, value_cache, slot_mapping, k_scale, v_scale, out_k, out_v, 1, num_tokens, \
                      num_blocks, num_heads, head_dim, block_size, dtype_code, 0, as_stream(stream));             \
  }                                                                                                               \
  int musa_aiter_kv_paged_fp8_to_linear_vec4_##FMT(                                                               \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, const float* k_scale,          \
      const float* v_scale, void* out_k, void* out_v, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,  \
      int64_t head_dim, int64_t block_size, int dtype_code, void* stream, int scale_mode) {                       \
    return fp8_gather(CODEC, key_cache, value_cache, slot_mapping, k_scale, v_scale, out_k, out_v, 1, num_tokens, \
                      num_blocks, num_heads, head_dim, block_size, dtype_code, scale_mode, as_stream(stream));    \
  }                                                                                                               \
  int musa_aiter_kv_linear_to_paged_fp8_multi_layer_##FMT(                                                        \
      const void* key_linear, const void* value_linear, const int64_t* slot_mapping, void* key_cache,             \
      void* value_cache, const float* k_scale, const float* v_scale, int64_t num_layers, int64_t num_tokens,      \
      int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size, int dtype_code, void* stream,  \
      int scale_mode) {                                                                                           \
    return fp8_scatter(CODEC, key_linear, value_linear, slot_mapping, key_cache, value_cache, k_scale, v_scale,   \
                       num_layers, num_tokens, num_blocks, num_heads, head_dim, block_size, dtype_code,           \
                       scale_mode, as_stream(stream));                                                            \
  }                                                                                                               \
  int musa_aiter_kv_paged_fp8_to_linear_multi_layer_##FMT(                                                        \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, const float* k_scale,          \
      const float* v_scale, void* out_k, void* out_v, int64_t num_layers, int64_t num_tokens, int64_t num_blocks, \
      int64_t num_heads, int64_t head_dim, int64_t block_size, int dtype_code, void* stream, int scale_mode) {    \
    return fp8_gather(CODEC, key_cache, value_cache, slot_mapping, k_scale, v_scale, out_k, out_v, num_layers,    \
                      num_tokens, num_blocks, num_heads, head_dim, block_size, dtype_code, scale_mode,            \
                      as_stream(stream));                                                                         \
  }

KVHIP_FP8(e4m3, kvhip::kE4M3)
KVHIP_FP8(e5m2, kvhip::kE5M2)
#undef KVHIP_FP8

// Shape-specialised gathers of the reference (scalar scale); one kernel family
// serves all of them here.
#define KVHIP_FP8_SHAPE(HD, BS, FMT, CODEC)                                                                        \
  int musa_aiter_kv_paged_fp8_to_linear_hd##HD##_bs##BS##_##FMT(                                                  \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, const float* k_scale,          \
      const float* v_scale, void* out_k, void* out_v, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,  \
      int dtype_code, void* stream) {                                                                             \
    return fp8_gather(CODEC, key_cache, value_cache, slot_mapping, k_scale, v_scale, out_k, out_v, 1, num_tokens, \
                      num_blocks, num_heads, HD, BS, dtype_code, 0, as_stream(stream));                           \
  }

KVHIP_FP8_SHAPE(64, 16, e4m3, kvhip::kE4M3)
KVHIP_FP8_SHAPE(64, 16, e5m2, kvhip::kE5M2)
KVHIP_FP8_SHAPE(128, 16, e4m3, kvhip::kE4M3)
KVHIP_FP8_SHAPE(128, 16, e5m2, kvhip::kE5M2)
KVHIP_FP8_SHAPE(128, 32, e4m3, kvhip::kE4M3)
KVHIP_FP8_SHAPE(128, 32, e5m2, kvhip::kE5M2)
#undef KVHIP_FP8_SHAPE

// ----- LMCache legacy 6-D and MLA (lmcache_kv_transfer.py:628-696) -----------------------------

#define KVHIP_LMCACHE_DENSE(SUFFIX, ELT)                                                                          \
  int lmcache_kv_buffer_to_paged##SUFFIX(const void* kv_buffer, void* paged_kv_cache, const int64_t* slot_mapping, \
                                         int64_t num_layers, int64_t num_tokens, int64_t num_blocks,               \
                                         int64_t block_size, int64_t num_heads, int64_t head_size, void* stream) { \
    return lmcache_6d(1, ELT, kv_buffer, paged_kv_cache, slot_mapping, num_layers, num_tokens, num_blocks,        \
                      block_size, num_heads, head_size, as_stream(stream));                                       \
  }                                                                                                               \
  int lmcache_paged_to_kv_buffer##SUFFIX(const void* paged_kv_cache, void* kv_buffer, const int64_t* slot_mapping, \
                                         int64_t num_layers, int64_t num_tokens, int64_t num_blocks,               \
                                         int64_t block_size, int64_t num_heads, int64_t head_size, void* stream) { \
    return lmcache_6d(0, ELT, kv_buffer, paged_kv_cache, slot_mapping, num_layers, num_tokens, num_blocks,        \
                      block_size, num_heads, head_size, as_stream(stream));                                       \
  }                                                                                                               \
  int lmcache_kv_buffer_to_paged_mla##SUFFIX(const void* kv_buffer, void* paged_kv_cache,                         \
                                             const int64_t* slot_mapping, int64_t num_layers, int64_t num_tokens, \
                                             int64_t num_blocks, int64_t block_size, int64_t hidden_size,         \
                                             void* stream) {                                                      \
    return lmcache_mla(1, ELT, kv_buffer, paged_kv_cache, slot_mapping, num_layers, num_tokens, num_blocks,       \
                       block_size, hidden_size, as_stream(stream));                                               \
  }                                                                                                               \
  int lmcache_paged_to_kv_buffer_mla##SUFFIX(const void* paged_kv_cache, void* kv_buffer,                         \
                                             const int64_t* slot_mapping, int64_t num_layers, int64_t num_tokens, \
                                             int64_t num_blocks, int64_t block_size, int64_t hidden_size,         \
                                             void* stream) {                                                      \
    return lmcache_mla(0, ELT, kv_buffer, paged_kv_cache, slot_mapping, num_layers, num_tokens, num_blocks,       \
                       block_size, hidden_size, as_stream(stream));                                               \
  }

KVHIP_LMCACHE_DENSE(, 4)
KVHIP_LMCACHE_DENSE(_u16, 2)
#undef KVHIP_LMCACHE_DENSE

// ----- LMCache SGLang-MP 2 x NL (lmcache_kv_transfer.py:713-761; kv_transfer_float.mu:2072-2156) --

#define KVHIP_TWO_X_NL(SUFFIX, ELT)                                                                               \
  int lmcache_kv_buffer_to_paged_two_x_nl_##SUFFIX(                                                               \
      const void* memory_tensor, void* cache, const int64_t* slot_mapping, int64_t kv_axis, int64_t layer_index,  \
      int64_t num_layers, int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix_n_tokens,                \
      int64_t num_blocks, int64_t block_size, int64_t num_heads, int64_t head_size, void* stream) {               \
    const uint64_t plane = addr(cache, 0);                                                                        \
    return lmcache_planes(1, ELT, memory_tensor, &plane, &kv_axis, &layer_index, 1, slot_mapping, num_layers,     \
                          memory_tokens, num_tokens, skip_prefix_n_tokens, num_blocks, block_size,                \
                          num_heads * head_size, 0, as_stream(stream));                                           \
  }                                                                                                               \
  int lmcache_paged_to_kv_buffer_two_x_nl_##SUFFIX(                                                               \
      void* memory_tensor, const void* cache, const int64_t* slot_mapping, int64_t kv_axis, int64_t layer_index,  \
      int64_t num_layers, int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix_n_tokens,                \
      int64_t num_blocks, int64_t block_size, int64_t num_heads, int64_t head_size, void* stream) {               \
    const uint64_t plane = addr(cache, 0);                                                                        \
    return lmcache_planes(0, ELT, memory_tensor, &plane, &kv_axis, &layer_index, 1, slot_mapping, num_layers,     \
                          memory_tokens, num_tokens, skip_prefix_n_tokens, num_blocks, block_size,                \
                          num_heads * head_size, 0, as_stream(stream));                                           \
  }

KVHIP_TWO_X_NL(float, 4)
KVHIP_TWO_X_NL(u16, 2)
#undef KVHIP_TWO_X_NL

int lmcache_kv_buffer_to_paged_two_x_nl_coalesced_u16(const void* memory_tensor, const uint64_t* cache_ptrs,
                                                      const int64_t* slot_mapping, int64_t num_layers,
                                                      int64_t memory_tokens, int64_t num_tokens,
                                                      int64_t skip_prefix_n_tokens, int64_t num_blocks,
                                                      int64_t block_size, int64_t num_heads, int64_t head_size,
                                                      void* stream) {
  if (num_layers <= 0) return hipSuccess;
  std::vector<int64_t> axes(2 * num_layers), layers(2 * num_layers);
  for (int64_t i = 0; i < 2 * num_layers; ++i) {
    axes[i] = i / num_layers;
    layers[i] = i % num_layers;
  }
  return lmcache_planes(1, 2, memory_tensor, cache_ptrs, axes.data(), layers.data(), 2 * num_layers, slot_mapping,
                        num_layers, memory_tokens, num_tokens, skip_prefix_n_tokens, num_blocks, block_size,
                        num_heads * head_size, 0, as_stream(stream));
}

int lmcache_paged_to_kv_buffer_two_x_nl_coalesced_u16(void* memory_tensor, const uint64_t* cache_ptrs,
                                                      const int64_t* slot_mapping, int64_t num_layers,
                                                      int64_t memory_tokens, int64_t num_tokens, int64_t num_blocks,
                                                      int64_t block_size, int64_t num_heads, int64_t head_size,
                                                      void* stream) {
  if (num_layers <= 0) return hipSuccess;
  std::vector<int64_t> axes(2 * num_layers), layers(2 * num_layers);
  for (int64_t i = 0; i < 2 * num_layers; ++i) {
    axes[i] = i / num_layers;
    layers[i] = i % num_layers;
  }
  return lmcache_planes(0, 2, memory_tensor, cache_ptrs, axes.data(), layers.data(), 2 * num_layers, slot_mapping,
                        num_layers, memory_tokens, num_tokens, 0, num_blocks, block_size, num_heads * head_size, 0,
                        as_stream(stream));
}

// ----- LMCache per-layer list caches [2, NB, BS, NH, HS] (lmcache_kv_transfer.py:874-993) ------

#define KVHIP_LIST(SUFFIX, ELT)                                                                                   \
  int lmcache_kv_buffer_to_paged_list_##SUFFIX(const void* memory_tensor, void* kvcache,                          \
                                               const int64_t* slot_mapping, int64_t layer_index,                  \
                                               int64_t num_layers, int64_t memory_tokens, int64_t num_tokens,     \
                                               int64_t skip_prefix, int64_t num_blocks, int64_t block_size,       \
                                               int64_t num_heads, int64_t head_size, void* stream) {              \
    const int64_t plane_bytes = num_blocks * block_size * num_heads * head_size * ELT;                            \
    const uint64_t planes[2] = {addr(kvcache, 0), addr(kvcache, plane_bytes)};                                    \
    const int64_t axes[2] = {0, 1}, layers[2] = {layer_index, layer_index};                                       \
    return lmcache_planes(1, ELT, memory_tensor, planes, axes, layers, 2, slot_mapping, num_layers,               \
                          memory_tokens, num_tokens, skip_prefix, num_blocks, block_size, num_heads * head_size,  \
                          0, as_stream(stream));                                                                  \
  }                                                                                                               \
  int lmcache_paged_to_kv_buffer_list_##SUFFIX(void* memory_tensor, const void* kvcache,                          \
                                               const int64_t* slot_mapping, int64_t layer_index,                  \
                                               int64_t num_layers, int64_t memory_tokens, int64_t num_tokens,     \
                                               int64_t skip_prefix, int64_t num_blocks, int64_t block_size,       \
                                               int64_t num_heads, int64_t head_size, void* stream) {              \
    const int64_t plane_bytes = num_blocks * block_size * num_heads * head_size * ELT;                            \
    const uint64_t planes[2] = {addr(kvcache, 0), addr(kvcache, plane_bytes)};                                    \
    const int64_t axes[2] = {0, 1}, layers[2] = {layer_index, layer_index};                                       \
    return lmcache_planes(0, ELT, memory_tensor, planes, axes, layers, 2, slot_mapping, num_layers,               \
                          memory_tokens, num_tokens, skip_prefix, num_blocks, block_size, num_heads * head_size,  \
                          0, as_stream(stream));                                                                  \
  }

KVHIP_LIST(float, 4)
KVHIP_LIST(u16, 2)
#undef KVHIP_LIST

static int list2(int scatter, const void* memory_tensor, const void* kvcache0, const void* kvcache1,
                 const int64_t* slot_mapping, int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix,
                 int64_t num_blocks, int64_t block_size, int64_t num_heads, int64_t head_size, void* stream) {
  const int64_t plane_bytes = num_blocks * block_size * num_heads * head_size * 2;
  const uint64_t planes[4] = {addr(kvcache0, 0), addr(kvcache1, 0), addr(kvcache0, plane_bytes),
                              addr(kvcache1, plane_bytes)};
  const int64_t axes[4] = {0, 0, 1, 1}, layers[4] = {0, 1, 0, 1};
  return lmcache_planes(scatter, 2, memory_tensor, planes, axes, layers, 4, slot_mapping, 2, memory_tokens,
                        num_tokens, skip_prefix, num_blocks, block_size, num_heads * head_size, 0,
                        as_stream(stream));
}

int lmcache_kv_buffer_to_paged_list2_u16(const void* memory_tensor, void* kvcache0, void* kvcache1,
                                         const int64_t* slot_mapping, int64_t memory_tokens, int64_t num_tokens,
                                         int64_t skip_prefix, int64_t num_blocks, int64_t block_size,
                                         int64_t num_heads, int64_t head_size, void* stream) {
  return list2(1, memory_tensor, kvcache0, kvcache1, slot_mapping, memory_tokens, num_tokens, skip_prefix,
               num_blocks, block_size, num_heads, head_size, stream);
}

int lmcache_paged_to_kv_buffer_list2_u16(void* memory_tensor, const void* kvcache0, const void* kvcache1,
                                         const int64_t* slot_mapping, int64_t memory_tokens, int64_t num_tokens,
                                         int64_t skip_prefix, int64_t num_blocks, int64_t block_size,
                                         int64_t num_heads, int64_t head_size, void* stream) {
  return list2(0, memory_tensor, kvcache0, kvcache1, slot_mapping, memory_tokens, num_tokens, skip_prefix,
               num_blocks, block_size, num_heads, head_size, stream);
}

// The reference extension's list2 kernel variants (lmcache_kv_transfer_ext.cpp:42-125) move the same
// bytes; they all run the list2 transfer above.
int lmcache_kv_buffer_to_paged_list2_u16_coalesced(const void* memory_tensor, void* kvcache0, void* kvcache1,
                                                   const int64_t* slot_mapping, int64_t memory_tokens,
                                                   int64_t num_tokens, int64_t skip_prefix, int64_t num_blocks,
                                                   int64_t block_size, int64_t num_heads, int64_t head_size,
                                                   void* stream) {
  return list2(1, memory_tensor, kvcache0, kvcache1, slot_mapping, memory_tokens, num_tokens, skip_prefix,
               num_blocks, block_size, num_heads, head_size, stream);
}

#define KVHIP_LIST2_GATHER_VARIANT(VARIANT)                                                                       \
  int lmcache_paged_to_kv_buffer_list2_u16_##VARIANT(void* memory_tensor, const void* kvcache0,                  \
                                                     const void* kvcache1, const int64_t* slot_mapping,           \
                                                     int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix, \
                                                     int64_t num_blocks, int64_t block_size, int64_t num_heads,   \
                                                     int64_t head_size, void* stream) {                           \
    return list2(0, memory_tensor, kvcache0, kvcache1, slot_mapping, memory_tokens, num_tokens, skip_prefix,      \
                 num_blocks, block_size, num_heads, head_size, stream);                                           \
  }
KVHIP_LIST2_GATHER_VARIANT(coalesced)
KVHIP_LIST2_GATHER_VARIANT(contiguous)
KVHIP_LIST2_GATHER_VARIANT(contiguous_bulk)
KVHIP_LIST2_GATHER_VARIANT(torchmusa_style)
#undef KVHIP_LIST2_GATHER_VARIANT

int lmcache_paged_to_kv_buffer_list2_u16_sorted(void* memory_tensor, const void* kvcache0, const void* kvcache1,
                                                const int64_t* slot_mapping, const uint8_t* /*sorted_indices_bytes*/,
                                                int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix,
                                                int64_t num_blocks, int64_t block_size, int64_t num_heads,
                                                int64_t head_size, void* stream) {
  return list2(0, memory_tensor, kvcache0, kvcache1, slot_mapping, memory_tokens, num_tokens, skip_prefix,
               num_blocks, block_size, num_heads, head_size, stream);
}

// ----- LMCache MLA list caches [NB, BS, HS] <-> [1, NL, M, HS] (lmcache_kv_transfer.py:920-950) -----

#define KVHIP_MLA_LIST(SUFFIX, ELT)                                                                               \
  int lmcache_mla_buffer_to_paged_list_##SUFFIX(const void* memory_tensor, void* kvcache,                         \
                                                const int64_t* slot_mapping, int64_t layer_index,                 \
                                                int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix,   \
                                                int64_t num_blocks, int64_t block_size, int64_t head_size,        \
                                                void* stream) {                                                   \
    const uint64_t plane = addr(kvcache, 0);                                                                      \
    const int64_t axis = 0;                                                                                       \
    return lmcache_planes(1, ELT, memory_tensor, &plane, &axis, &layer_index, 1, slot_mapping, 1, memory_tokens,  \
                          num_tokens, skip_prefix, num_blocks, block_size, head_size, 0, as_stream(stream));      \
  }                                                                                                               \
  int lmcache_mla_paged_to_buffer_list_##SUFFIX(void* memory_tensor, const void* kvcache,                         \
                                                const int64_t* slot_mapping, int64_t layer_index,                 \
                                                int64_t memory_tokens, int64_t num_tokens, int64_t num_blocks,    \
                                                int64_t block_size, int64_t head_size, void* stream) {            \
    const uint64_t plane = addr(kvcache, 0);                                                                      \
    const int64_t axis = 0;                                                                                       \
    return lmcache_planes(0, ELT, memory_tensor, &plane, &axis, &layer_index, 1, slot_mapping, 1, memory_tokens,  \
                          num_tokens, 0, num_blocks, block_size, head_size, 0, as_stream(stream));                \
  }

KVHIP_MLA_LIST(float, 4)
KVHIP_MLA_LIST(half, 2)
KVHIP_MLA_LIST(bfloat16, 2)
KVHIP_MLA_LIST(u16, 2)
#undef KVHIP_MLA_LIST

// ----- DSV4 opaque byte rows (kv_transfer.py:4209-4406) --------------------------------------------

int musa_aiter_kv_copy_paged_rows_u8(const void* src, void* dst, const int64_t* src_indices,
                                     const int64_t* dst_indices, int64_t num_rows, int64_t item_bytes,
                                     int64_t src_num_rows, int64_t dst_num_rows, void* stream) {
  const uint64_t s = addr(src, 0), d = addr(dst, 0);
  return musa_aiter_hip_copy_rows(&s, &d, nullptr, nullptr, 1, src_indices, dst_indices, num_rows, num_rows, 0, 0,
                                  src_num_rows, dst_num_rows, item_bytes, item_bytes, item_bytes, 0, 1, nullptr,
                                  stream);
}

int musa_aiter_kv_copy_paged_rows_layer_table_u8(const uint64_t* src_ptr_table, const uint64_t* dst_ptr_table,
                                                 const int64_t* src_indices, const int64_t* dst_indices,
                                                 int64_t num_rows, int64_t item_bytes, int64_t num_layers,
                                                 int64_t src_num_rows, int64_t dst_num_rows, void* stream) {
  return musa_aiter_hip_copy_rows(nullptr, nullptr, src_ptr_table, dst_ptr_table, num_layers, src_indices,
                                  dst_indices, num_rows, num_rows, 0, 0, src_num_rows, dst_num_rows, item_bytes,
                                  item_bytes, item_bytes, 0, 1, nullptr, stream);
}

int musa_aiter_kv_copy_paged_rows_contig_layers_u8(const void* src_base, void* dst_base, const int64_t* src_indices,
                                                   const int64_t* dst_indices, int64_t num_rows, int64_t item_bytes,
                                                   int64_t num_layers, int64_t src_num_rows, int64_t dst_num_rows,
                                                   void* stream) {
  if (num_layers <= 0) return hipSuccess;
  std::vector<uint64_t> s(num_layers), d(num_layers);
  for (int64_t l = 0; l < num_layers; ++l) {
    s[l] = addr(src_base, l * src_num_rows * item_bytes);
    d[l] = addr(dst_base, l * dst_num_rows * item_bytes);
  }
  return musa_aiter_hip_copy_rows(s.data(), d.data(), nullptr, nullptr, num_layers, src_indices, dst_indices,
                                  num_rows, num_rows, 0, 0, src_num_rows, dst_num_rows, item_bytes, item_bytes,
                                  item_bytes, 0, 1, nullptr, stream);
}

// ----- LMCache DSV4 strided block transfer (lmcache_kv_transfer.py:1355-1400) ----------------------

int lmcache_kv_strided_block_transfer(void* staging, const uint64_t* paged_ptrs, const int64_t* block_ids,
                                      int64_t direction, int64_t num_layers, int64_t idx_start, int64_t n_valid,
                                      int64_t offset_in_object, int64_t staging_tokens, int64_t block_size,
                                      int64_t row_bytes, int64_t paged_block_stride, int64_t mode,
                                      int64_t value_bytes, int64_t scale_bytes, void* stream) {
  kvhip::StridedBlockParams p{};
  p.staging = static_cast<uint8_t*>(staging);
  p.paged_ptrs = paged_ptrs;
  p.block_ids = block_ids;
  p.direction = direction;
  p.num_layers = num_layers;
  p.idx_start = idx_start;
  p.n_valid = n_valid;
  p.offset_in_object = offset_in_object;
  p.staging_tokens = staging_tokens;
  p.block_size = block_size;
  p.row_bytes = row_bytes;
  p.paged_block_stride = paged_block_stride;
  p.mode = mode;
  p.value_bytes = value_bytes;
  p.scale_bytes = scale_bytes;
  return kvhip::launch_strided_blocks(p, as_stream(stream));
}

// ----- SGLang HiCache transfers (hicache_transfer.mu:53-98, hicache_transfer.py:190-258) ---------

int musa_aiter_hicache_transfer_abi_version() { return 1; }

// Rows copied between two index-addressed sides whose planes are listed on
// the host; either side may use paged row addressing.  Tokens whose source or
// destination index lies outside [0, rows) are skipped; with `dedupe` a
// destination row named by several tokens keeps the last one.
int musa_aiter_hip_copy_rows_paged(const uint64_t* src_planes, const uint64_t* dst_planes, int64_t num_planes,
                                   const int64_t* src_idx, const int64_t* dst_idx, int64_t num_tokens,
                                   int64_t src_rows, int64_t dst_rows, int64_t row_bytes, int64_t src_stride,
                                   int64_t dst_stride, int64_t src_page_rows, int64_t src_page_stride,
                                   int64_t dst_page_rows, int64_t dst_page_stride, int dedupe,
                                   const musa_aiter_hip_claims* claims, void* stream) {
  if (num_tokens <= 0 || num_planes <= 0 || row_bytes <= 0) return hipSuccess;
  if (src_idx == nullptr || dst_idx == nullptr) return hipErrorInvalidValue;
  RowCopyParams p{};
  p.src_planes = src_planes;
  p.dst_planes = dst_planes;
  p.num_planes = num_planes;
  p.src_idx = src_idx;
  p.dst_idx = dst_idx;
  p.num_tokens = num_tokens;
  p.num_rows_out = num_tokens;
  p.src_rows = src_rows;
  p.dst_rows = dst_rows;
  p.row_bytes = row_bytes;
  p.src_stride = src_stride;
  p.dst_stride = dst_stride;
  p.src_page_rows = src_page_rows;
  p.src_page_stride = src_page_stride;
  p.dst_page_rows = dst_page_rows;
  p.dst_page_stride = dst_page_stride;
  if (dedupe) {
    kvhip::ClaimSource src;
    src.idx = dst_idx;
    src.src_idx = src_idx;
    src.src_rows = src_rows;
    hipError_t err =
        prepare_claims(src, num_tokens, dst_rows, as_stream(stream), claims, &p.owner, &p.epoch, &p.owner_exclusive);
    if (err != hipSuccess) return err;
  }
  return kvhip::launch_row_copy(p, as_stream(stream));
}

// The reference kernel's contract: for every item whose two page indices are
// both non-negative and every layer in [start_layer, start_layer + num_layers),
// item_size_bytes (whole 64-bit words) move from
// src + page * src_page_stride + layer * src_layer_stride to the matching
// destination offset, for K and, when both V pointers are set, for V.  Page
// indices are not range-checked (the caller validates them) and a destination
// page named by several items receives one of them.
int musa_aiter_hicache_transfer_bytes(const void* src_k, void* dst_k, const void* src_v, void* dst_v,
                                      const int64_t* src_indices, const int64_t* dst_indices, int64_t num_items,
                                      int64_t start_layer, int64_t num_layers, int64_t item_size_bytes,
                                      int64_t src_page_stride_bytes, int64_t src_layer_stride_bytes,
                                      int64_t dst_page_stride_bytes, int64_t dst_layer_stride_bytes, void* stream) {
  const int64_t row = item_size_bytes / 8 * 8;
  if (num_items <= 0 || num_layers <= 0 || row <= 0) return hipSuccess;
  if (src_k == nullptr || dst_k == nullptr || src_indices == nullptr || dst_indices == nullptr)
    return hipErrorInvalidValue;
  const bool with_v = src_v != nullptr && dst_v != nullptr;
  std::vector<uint64_t> s, d;
  for (int kv = 0; kv < (with_v ? 2 : 1); ++kv)
    for (int64_t l = 0; l < num_layers; ++l) {
      s.push_back(addr(kv == 0 ? src_k : src_v, (start_layer + l) * src_layer_stride_bytes));
      d.push_back(addr(kv == 0 ? dst_k : dst_v, (start_layer + l) * dst_layer_stride_bytes));
    }
  const int64_t unbounded = INT64_MAX;
  return musa_aiter_hip_copy_rows_paged(s.data(), d.data(), static_cast<int64_t>(s.size()), src_indices,
                                        dst_indices, num_items, unbounded, unbounded, row, src_page_stride_bytes,
                                        dst_page_stride_bytes, 0, 0, 0, 0, 0, nullptr, stream);
}

// ----- LMCache host <-> device batch copies (lmcache_musa_batch_copy_ext.cpp:41-277) -------------

int musa_aiter_hip_batch_copy_abi_version() { return 1; }

int musa_aiter_hip_runtime_versions(int* runtime_version, int* driver_version) {
  if (runtime_version == nullptr || driver_version == nullptr) return hipErrorInvalidValue;
  const hipError_t err = hipRuntimeGetVersion(runtime_version);
  if (err != hipSuccess) return err;
  return hipDriverGetVersion(driver_version);
}

// Byte ranges between pinned or pageable host memory and device memory of the
// current device, all in one direction (0: host -> device, 1: device -> host),
// submitted on `stream`.  mode 0 and 1: ranges whose host side is pinned host
// memory with a device mapping go through the batch-copy kernel (one launch for
// the whole batch) on at most kBatchGroups (mode 0) or kOverlapGroups workgroups (mode 1,
// which leaves nearly all compute units to concurrent kernels); the other
// ranges go through hipMemcpyAsync.  mode 2: every range goes through
// hipMemcpyAsync.  Measured on MI355X, a few dozen workgroups keep enough
// requests in flight for the host link, and fewer contend less: 16-64
// workgroups move 512 KiB ranges at 54-57 GB/s against 52-53 GB/s with one
// workgroup per tile, while 4 KiB ranges need at least 32.
constexpr uint32_t kBatchGroups = 64;
constexpr uint32_t kOverlapGroups = 16;

// Batches of more than kBatchCopyMax ranges take one launch over per-tile
// descriptors written into pinned host memory.  Each (device, stream) has a
// ring of kDescSlots such buffers; a slot is rewritten only after the event
// recorded behind its last launch has completed, so several batches can be
// queued on the stream without waiting.
constexpr int kDescSlots = 4;

struct DescSlot {
  uint64_t* host = nullptr;
  size_t capacity = 0;  // uint64 values
  hipEvent_t done = nullptr;
  bool pending = false;
};

struct DescRing {
  std::mutex mu;  // held while a slot is claimed, waited for and refilled
  DescSlot slots[kDescSlots];
  int next = 0;
};

// g_desc_mu guards only the ring lookup; waits happen under the ring's own
// mutex, so batches on other streams never queue behind them.
std::mutex g_desc_mu;
std::map<std::pair<int, uintptr_t>, DescRing>* g_desc_rings = nullptr;
// Outgrown descriptor buffers: freeing pinned memory synchronises the device,
// so they stay allocated (capacities double, bounding them by the live ones).
std::vector<uint64_t*>* g_retired_desc = nullptr;

hipError_t batch_copy_by_descriptors(const std::vector<uint64_t>& src, const std::vector<uint64_t>& dst,
                                     const std::vector<uint64_t>& size, uint32_t max_groups, hipStream_t stream) {
  const uint64_t tiles = kvhip::batch_copy_tile_count(size.data(), static_cast<int64_t>(size.size()));
  if (tiles == 0) return hipSuccess;
  if (tiles > 0x7FFFFFFFu) return hipErrorInvalidValue;
  int dev = 0;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return err;
  DescRing* ring_ptr = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_desc_mu);
    if (g_desc_rings == nullptr) g_desc_rings = new std::map<std::pair<int, uintptr_t>, DescRing>();
    ring_ptr = &(*g_desc_rings)[{dev, reinterpret_cast<uintptr_t>(stream)}];  // map nodes never move
  }
  DescRing& ring = *ring_ptr;
  std::lock_guard<std::mutex> ring_lock(ring.mu);
  DescSlot& slot = ring.slots[ring.next];
  ring.next = (ring.next + 1) % kDescSlots;
  if (slot.pending) {
    err = hipEventSynchronize(slot.done);
    if (err != hipSuccess) return err;
    slot.pending = false;
  }
  if (slot.done == nullptr) {
    err = hipEventCreateWithFlags(&slot.done, hipEventDisableTiming);
    if (err != hipSuccess) {
      slot.done = nullptr;
      return err;
    }
  }
  const size_t need = static_cast<size_t>(tiles) * 3;
  if (slot.capacity < need) {
    size_t cap = slot.capacity * 2;
    if (cap < need) cap = need;
    if (cap < 8192) cap = 8192;
    uint64_t* host = nullptr;
    err = hipHostMalloc(reinterpret_cast<void**>(&host), cap * sizeof(uint64_t),
                        hipHostMallocMapped | hipHostMallocCoherent);
    if (err != hipSuccess) return err;
    g_allocated_bytes.fetch_add(static_cast<int64_t>(cap * sizeof(uint64_t)));
    if (slot.host != nullptr) {
      std::lock_guard<std::mutex> lock(g_desc_mu);
      if (g_retired_desc == nullptr) g_retired_desc = new std::vector<uint64_t*>();
      g_retired_desc->push_back(slot.host);
    }
    slot.host = host;
    slot.capacity = cap;
  }
  kvhip::batch_copy_fill_desc(src.data(), dst.data(), size.data(), static_cast<int64_t>(size.size()), slot.host);
  void* mapped = nullptr;
  err = hipHostGetDevicePointer(&mapped, slot.host, 0);
  if (err != hipSuccess) return err;
  err = kvhip::launch_batch_copy_desc(static_cast<const uint64_t*>(mapped), tiles, max_groups, stream);
  if (err != hipSuccess) return err;
  err = hipEventRecord(slot.done, stream);
  if (err != hipSuccess) return err;
  slot.pending = true;
  return hipSuccess;
}

// The last pinned host allocation seen in one batch call: host range [lo, hi) and
// the device address of lo.  Batches usually take many ranges from one staging
// buffer, so one range lookup replaces a pointer query per range.
struct PinnedRange {
  uint64_t lo = 0, hi = 0, dev = 0;
};

// Device-side address of `host` when it lies in pinned host memory with a
// device mapping.  A pointer outside the cached range is queried; its
// allocation's range is then cached, but only when the device address of the
// range's last byte, queried on its own, lies at the same offset.
bool map_pinned(const void* host, PinnedRange& cache, uint64_t* mapped) {
  const uint64_t h = reinterpret_cast<uint64_t>(host);
  if (h >= cache.lo && h < cache.hi) {
    *mapped = cache.dev + (h - cache.lo);
    return true;
  }
  auto query = [](const void* p, uint64_t* dev) {
    hipPointerAttribute_t attr{};
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
      (void)hipGetLastError();  // pageable memory: clear the query's error
      return false;
    }
    if (attr.type != hipMemoryTypeHost || attr.devicePointer == nullptr || attr.hostPointer == nullptr) return false;
    *dev = reinterpret_cast<uint64_t>(attr.devicePointer) +
           (reinterpret_cast<uint64_t>(p) - reinterpret_cast<uint64_t>(attr.hostPointer));
    return true;
  };
  if (!query(host, mapped)) return false;
  void* start = nullptr;
  size_t size = 0;
  hipDeviceptr_t hp = const_cast<void*>(host);
  if (hipPointerGetAttribute(&start, HIP_POINTER_ATTRIBUTE_RANGE_START_ADDR, hp) != hipSuccess ||
      hipPointerGetAttribute(&size, HIP_POINTER_ATTRIBUTE_RANGE_SIZE, hp) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  const uint64_t lo = reinterpret_cast<uint64_t>(start);
  if (size == 0 || h < lo || h - lo >= size) return true;
  const uint64_t dev_lo = *mapped - (h - lo);
  uint64_t dev_last = 0;
  if (query(reinterpret_cast<const void*>(lo + size - 1), &dev_last) && dev_last == dev_lo + (size - 1))
    cache = PinnedRange{lo, lo + size, dev_lo};
  return true;
}

int musa_aiter_hip_batch_copy(void* const* dsts, const void* const* srcs, const uint64_t* sizes, int64_t count,
                              int direction, int mode, void* stream) {
  if (count <= 0) return hipSuccess;
  if (dsts == nullptr || srcs == nullptr || sizes == nullptr || (direction != 0 && direction != 1) || mode < 0 ||
      mode > 2)
    return hipErrorInvalidValue;
  const bool use_copy_engines = mode == 2;
  const hipMemcpyKind kind = direction == 0 ? hipMemcpyHostToDevice : hipMemcpyDeviceToHost;
  std::vector<uint64_t> ks, kd, kn;
  ks.reserve(static_cast<size_t>(count));
  kd.reserve(static_cast<size_t>(count));
  kn.reserve(static_cast<size_t>(count));
  PinnedRange pinned;
  for (int64_t i = 0; i < count; ++i) {
    if (sizes[i] == 0) continue;
    if (dsts[i] == nullptr || srcs[i] == nullptr) return hipErrorInvalidValue;
    const void* host = direction == 0 ? srcs[i] : dsts[i];
    uint64_t mapped = 0;
    const bool kernel = !use_copy_engines && map_pinned(host, pinned, &mapped);
    if (kernel) {
      ks.push_back(direction == 0 ? mapped : reinterpret_cast<uint64_t>(srcs[i]));
      kd.push_back(direction == 0 ? reinterpret_cast<uint64_t>(dsts[i]) : mapped);
      kn.push_back(sizes[i]);
    } else {
      const hipError_t err = hipMemcpyAsync(dsts[i], srcs[i], sizes[i], kind, as_stream(stream));
      if (err != hipSuccess) return err;
    }
  }
  const uint32_t groups = mode == 1 ? kOverlapGroups : kBatchGroups;
  if (ks.size() > static_cast<size_t>(kvhip::kBatchCopyMax)) {
    // A graph capture would keep the descriptor slot's address while the ring
    // reuses it, so captured batches stay on the kernel-argument launches.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    const hipError_t err = hipStreamIsCapturing(as_stream(stream), &capture);
    if (err != hipSuccess) return err;
    if (capture == hipStreamCaptureStatusNone) return batch_copy_by_descriptors(ks, kd, kn, groups, as_stream(stream));
  }
  return kvhip::launch_batch_copy(ks.data(), kd.data(), kn.data(), static_cast<int64_t>(ks.size()), groups,
                                  as_stream(stream));
}

// ----- CacheGen-style codec (kv_transfer_float.mu:828-898, kv_transfer.py:1048-1215) ----------

int musa_aiter_kv_cachegen_encode_float(const void* input, void* encoded, float min_val, float scale, int64_t numel,
                                        int64_t num_bins, void* stream) {
  if (numel <= 0) return hipSuccess;
  if (input == nullptr || encoded == nullptr || num_bins < 1 || num_bins > 256) return hipErrorInvalidValue;
  return kvhip::launch_cachegen_bins(static_cast<const float*>(input), static_cast<uint8_t*>(encoded), min_val, scale,
                                     numel, static_cast<int>(num_bins), as_stream(stream));
}

int musa_aiter_kv_cachegen_decode_float(const void* encoded, const void* codebook, void* output, int64_t numel,
                                        void* stream) {
  if (numel <= 0) return hipSuccess;
  if (encoded == nullptr || codebook == nullptr || output == nullptr) return hipErrorInvalidValue;
  return kvhip::launch_cachegen_decode(static_cast<const uint8_t*>(encoded), numel, codebook, -1, 4, output, nullptr,
                                       as_stream(stream));
}

int64_t musa_aiter_hip_cachegen_workspace_bytes(void) { return kvhip::kCacheGenWorkspaceBytes; }

int musa_aiter_hip_cachegen_encode(const void* input, int input_dtype, int64_t numel, int64_t num_bins,
                                   int native_rounding, void* encoded, void* codebook, void* cdf, void* workspace,
                                   int64_t workspace_bytes, void* stream) {
  if (numel <= 0) return hipSuccess;
  if (input == nullptr || encoded == nullptr || codebook == nullptr || cdf == nullptr || workspace == nullptr ||
      num_bins < 2 || num_bins > 256 || workspace_bytes < kvhip::kCacheGenWorkspaceBytes ||
      (native_rounding != 0 && input_dtype != kvhip::kCgF32))
    return hipErrorInvalidValue;
  return kvhip::launch_cachegen_encode(input, input_dtype, numel, static_cast<int>(num_bins), native_rounding != 0,
                                       static_cast<uint8_t*>(encoded), static_cast<float*>(codebook),
                                       static_cast<float*>(cdf), workspace, as_stream(stream));
}

int musa_aiter_hip_cachegen_decode(const void* encoded, int64_t numel, const void* table, int64_t table_len,
                                   int elem_bytes, void* output, int32_t* max_code, void* stream) {
  if (numel <= 0) return hipSuccess;
  if (encoded == nullptr || table == nullptr || output == nullptr || table_len < 1 || table_len > 256 ||
      reinterpret_cast<uintptr_t>(table) % static_cast<uintptr_t>(elem_bytes > 0 ? elem_bytes : 1) != 0)
    return hipErrorInvalidValue;
  return kvhip::launch_cachegen_decode(static_cast<const uint8_t*>(encoded), numel, table, static_cast<int>(table_len),
                                       elem_bytes, output, max_code, as_stream(stream));
}

}  // extern "C"
