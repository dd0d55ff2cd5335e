/*
 * C-ABI of libmusa_aiter_kv_hip.so -- MI355X (gfx950) KV-cache movement kernels.
 *
 * Every function below is exported with C linkage, takes plain pointers
 * (device addresses unless noted) and 64-bit sizes, launches asynchronously
 * on `stream` (a hipStream_t passed as void*; NULL = the default stream) and
 * returns the HIP status as an int (0 = success).  Names and argument orders
 * are the ones the reference (musa_aiter 0.5.0) binds through ctypes, cited
 * per entry as file:line of the reference's musa_aiter/ops Python modules (the
 * binding) and of its csrc/kvcache .mu sources (the symbol it replaces).  A reference build that binds
 * these names with restype=None keeps working; binding restype=c_int gives
 * the launch status.
 *
 * Conventions shared by all entries:
 *   slot = block * block_size + offset; slot < 0 skips the token (gathers
 *   write zeros, scatters leave the destination untouched); slots outside
 *   the cache are treated as skipped.  Scatters keep last-writer-wins for
 *   duplicate destinations, like the reference's token loop: a claim pass
 *   records the last token per destination in a tag array: the caller's
 *   (generic entries given musa_aiter_hip_claims), or one the library owns
 *   per (device, stream) (allocated on first use, grown on demand; calls
 *   captured into a HIP graph get an array per capture and stream, reused
 *   once that graph is destroyed).
 *   Element types: "_float" = fp32, "_half" = fp16, "_bfloat16" / "_u16" =
 *   16-bit payloads (bf16 or fp16, copied bit-exactly).
 */
#ifndef MUSA_AITER_KV_HIP_H_
#define MUSA_AITER_KV_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- ABI probes (kv_transfer_float.mu:3021-3027, :3277; fp8_kv_cache.mu:1529-1531) ---- */
int musa_aiter_kv_transfer_abi_version(void);
int native_lmcache_kv_transfer_abi_version(void);
int musa_aiter_fp8_kv_cache_abi_version(void);
int musa_aiter_dsv4_kv_copy_abi_version(void);
/* No reference counterpart: backend label and HIP error text for diagnostics. */
const char* musa_aiter_hip_backend_name(void);
const char* musa_aiter_hip_error_string(int code);
/* No reference counterpart: number of duplicate-slot claim arrays the library has allocated for
 * scatters captured into HIP graphs.  Each capture (and capturing stream) takes one; an array
 * returns to a free list when the graph that holds it is destroyed, and later captures reuse it,
 * so the count follows the number of graphs alive at once, not the number ever captured. */
int64_t musa_aiter_hip_graph_claim_arrays(void);
/* No reference counterpart: bytes of device and pinned host memory the library has allocated
 * itself since it was loaded (duplicate-slot claim arrays of the reference-named scatter entries,
 * descriptor rings of large host batches; the static array of musa_aiter_hip_paged_tiles_noalloc
 * is not counted).  The generic entries below allocate nothing when given caller-owned claims. */
int64_t musa_aiter_hip_allocated_bytes(void);
/* No reference counterpart: the largest entry of an int64 index vector, for the Python layer's
 * host-side bounds checks (the reference reads slot_mapping.max() with torch, kv_transfer.py:3024).
 * Launches `parts` (1-4096) workgroups on `stream`; workgroup w writes the maximum of the entries it
 * visits to partial[w] (INT64_MIN if none) and then `stamp` (nonzero, a value the caller changes per
 * call) to partial[parts + w].  `partial` (2 * parts entries) is pinned host memory the caller owns;
 * the call returns once every stamp is there (after at most 0.2 s of polling it synchronises the
 * stream instead), so the maxima can be read right after it; n >= 1. */
int musa_aiter_hip_index_max(const int64_t* idx, int64_t n, int64_t* partial, int64_t parts, int64_t stamp,
                             void* stream);
/* No reference counterpart: the access-pattern ceiling of a paged copy, timed by bench.py.  Copies
 * num_blocks whole blocks of every plane: block i reads block src_blocks[i] (NULL: i) of the source
 * region and writes block dst_blocks[i] (NULL: i) of the destination; block sizes are multiples of
 * 1 KiB, equal or in a 2:1 / 1:2 ratio (FP8 quant-store / dequant-gather traffic); ids outside
 * [0, *_region_blocks) are skipped.  int32 block ids; strides in bytes.  write_through: 0 non-temporal
 * stores, 1 also agent-scope (written through the L2, as the paged gathers' linear stores). */
int musa_aiter_hip_block_pattern_copy(const void* src, void* dst, const int32_t* src_blocks,
                                      const int32_t* dst_blocks, int64_t num_blocks, int64_t src_region_blocks,
                                      int64_t dst_region_blocks, int64_t src_block_bytes, int64_t dst_block_bytes,
                                      int64_t planes, int64_t src_plane_stride, int64_t dst_plane_stride,
                                      int write_through, void* stream);

/* ---- Generic entries used by this package's Python host layer (no reference counterpart) ----
 * Caller-owned duplicate-slot claim tags for the generic scatter entries.  With `claims` NULL a
 * scatter uses an array the library allocates per (device, stream); the Python host layer passes
 * a tensor from torch's caching allocator instead, so the library allocates nothing on that path.
 *   tags:     `capacity` uint64 on the call's device; capacity >= the destination rows of the call
 *             (otherwise the call returns hipErrorInvalidValue and launches nothing).
 *   epoch 0:  the call first clears the tags its tokens compete for, then claims; nothing is assumed
 *             of the array's contents (for calls captured into graphs, whose replays repeat it).
 *   epoch k:  every tag in the array was written with an epoch below k (a zeroed array, then
 *             epochs 1, 2, .. one per call); no clearing pass.
 * Calls that share an array must be ordered (one stream). */
typedef struct musa_aiter_hip_claims {
  uint64_t* tags;
  int64_t capacity;
  uint32_t epoch;
  uint32_t reserved;
} musa_aiter_hip_claims;

/* Paged-A caches [NL, NB, NH, HD, BS] <-> linear rows with explicit strides.
 * scatter: 0 gather, 1 scatter; codec: 0 copy, 1 FP8 E4M3, 2 FP8 E5M2;
 * cache_elt / lin_elt: element bytes; lin_dtype (FP8 only): 0 f32, 1 f16, 2 bf16;
 * lin_token_stride / lin_layer_stride in linear elements; scale_mode: 0 scalar,
 * 1 [NH], 2 [NL, NH]; fill_zeros: gather writes zeros for skipped tokens;
 * dedupe: scatter runs the last-writer claim pass; claims: caller-owned tags or NULL. */
int musa_aiter_hip_paged_tiles(int scatter, int codec, int cache_elt, int lin_elt, int lin_dtype, void* key_cache,
                               void* value_cache, void* key_linear, void* value_linear, const int64_t* slot_mapping,
                               int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,
                               int64_t head_dim, int64_t block_size, int64_t lin_token_stride,
                               int64_t lin_layer_stride, const float* k_scale, const float* v_scale, int scale_mode,
                               int fill_zeros, int dedupe, const musa_aiter_hip_claims* claims, void* stream);
/* No reference counterpart.  For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): musa_aiter_hip_paged_tiles with the
 * same arguments (but no `claims`) and results, allocating nothing.  A scatter with dedupe keeps
 * its last-writer claim tags in a static device array of MUSA_AITER_HIP_NOALLOC_MAX_SLOTS uint64 entries (16 MiB per
 * device, held until the process ends), cleared and claimed by every call; a scatter with dedupe
 * whose num_blocks * block_size exceeds that maximum returns hipErrorInvalidValue (1) and launches
 * nothing.  All calls on one device share the array: calls that overlap in time on one device
 * (concurrent streams, or graphs replaying at once) race and must not be issued. */
#define MUSA_AITER_HIP_NOALLOC_MAX_SLOTS 2097152
int musa_aiter_hip_paged_tiles_noalloc(int scatter, int codec, int cache_elt, int lin_elt, int lin_dtype,
                                       void* key_cache, void* value_cache, void* key_linear, void* value_linear,
                                       const int64_t* slot_mapping, int64_t num_layers, int64_t num_tokens,
                                       int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size,
                                       int64_t lin_token_stride, int64_t lin_layer_stride, const float* k_scale,
                                       const float* v_scale, int scale_mode, int fill_zeros, int dedupe,
                                       void* stream);
/* Paged-A caches [NB, NH, HD, BS] <-> dense [batch, dense_len, NH, HD] tensors addressed through
 * block tables: dense token (b, pos) uses slot block_tables[b, pos / BS] * BS + pos % BS while
 * pos < seq_lens[b], the logical block is below max_blocks and the block id lies in [0, num_blocks).
 * Same codec / element / scale / fill / dedupe arguments as musa_aiter_hip_paged_tiles;
 * dense_token_stride in dense elements.  batch * dense_len must stay below 2^31. */
int musa_aiter_hip_paged_dense_tiles(int scatter, int codec, int cache_elt, int lin_elt, int lin_dtype,
                                     void* key_cache, void* value_cache, void* dense_k, void* dense_v,
                                     const int64_t* block_tables, const int64_t* seq_lens, int64_t batch,
                                     int64_t dense_len, int64_t max_blocks, int64_t num_blocks, int64_t num_heads,
                                     int64_t head_dim, int64_t block_size, int64_t dense_token_stride,
                                     const float* k_scale, const float* v_scale, int scale_mode, int fill_zeros,
                                     int dedupe, const musa_aiter_hip_claims* claims, void* stream);
/* Dense [batch, dense_len, row_bytes] rows gathered from token-major caches [num_tokens, row_bytes]
 * through CSR indices (kv_indptr [batch + 1], kv_indices [index_count]); the byte-row form of
 * musa_aiter_kv_triton_indexed_to_dense_* for any element type. */
int musa_aiter_hip_csr_dense_rows(const void* key_cache, const void* value_cache, const int64_t* kv_indptr,
                                  const int64_t* kv_indices, void* out_k, void* out_v, int64_t batch,
                                  int64_t dense_len, int64_t index_count, int64_t num_tokens, int64_t row_bytes,
                                  void* stream);
/* Row copies between plane sets: planes given as host arrays (src_planes/dst_planes)
 * or device arrays (src_table/dst_table); a side is indexed through src_idx/dst_idx
 * or addressed directly (row = token + offset).  zero_invalid zero-fills directly
 * addressed destination rows whose source is skipped, and rows [num_tokens, num_rows_out). */
int musa_aiter_hip_copy_rows(const uint64_t* src_planes, const uint64_t* dst_planes, const uint64_t* src_table,
                             const uint64_t* dst_table, int64_t num_planes, const int64_t* src_idx,
                             const int64_t* dst_idx, int64_t num_tokens, int64_t num_rows_out, int64_t src_offset,
                             int64_t dst_offset, int64_t src_rows, int64_t dst_rows, int64_t row_bytes,
                             int64_t src_stride, int64_t dst_stride, int zero_invalid, int dedupe,
                             const musa_aiter_hip_claims* claims, void* stream);
/* musa_aiter_hip_copy_rows with its arguments in one struct (no reference counterpart; for the
 * Python host layer, which fills the struct with one struct.pack instead of converting 19
 * ctypes arguments, about 1.5 us less host time per call).  Fields as in musa_aiter_hip_copy_rows. */
typedef struct musa_aiter_hip_copy_rows_call {
  const uint64_t* src_planes;
  const uint64_t* dst_planes;
  const uint64_t* src_table;
  const uint64_t* dst_table;
  int64_t num_planes;
  const int64_t* src_idx;
  const int64_t* dst_idx;
  int64_t num_tokens;
  int64_t num_rows_out;
  int64_t src_offset;
  int64_t dst_offset;
  int64_t src_rows;
  int64_t dst_rows;
  int64_t row_bytes;
  int64_t src_stride;
  int64_t dst_stride;
  int32_t zero_invalid;
  int32_t dedupe;
  const musa_aiter_hip_claims* claims;
} musa_aiter_hip_copy_rows_call;
int musa_aiter_hip_copy_rows_packed(const musa_aiter_hip_copy_rows_call* call, void* stream);
/* Row copies between two index-addressed plane sets (host arrays of plane bases).  A side
 * with page_rows > 0 is paged: row r sits at (r / page_rows) * page_stride + (r % page_rows) *
 * stride of its plane (the page-first [pages, layers, page, item] tensors of SGLang's direct
 * HiCache transfers).  Tokens with an index outside [0, rows) are skipped; dedupe keeps the
 * last token of a repeated destination. */
int musa_aiter_hip_copy_rows_paged(const uint64_t* src_planes, const uint64_t* dst_planes, int64_t num_planes,
                                   const int64_t* src_idx, const int64_t* dst_idx, int64_t num_tokens,
                                   int64_t src_rows, int64_t dst_rows, int64_t row_bytes, int64_t src_stride,
                                   int64_t dst_stride, int64_t src_page_rows, int64_t src_page_stride,
                                   int64_t dst_page_rows, int64_t dst_page_stride, int dedupe,
                                   const musa_aiter_hip_claims* claims, void* stream);
/* Whole blocks copied between same-layout caches of num_layers layers (block_bytes per block and
 * layer, blocks contiguous per layer; K and V): block_mapping holds [num_pairs, 2] int64 (source,
 * destination) block ids; a pair with an id outside its cache is skipped, and a destination named
 * by several pairs keeps the last one.  The byte form of musa_aiter_kv_copy_paged_blocks_* with
 * caller-owned claims. */
int musa_aiter_hip_copy_blocks(const void* src_k, const void* src_v, void* dst_k, void* dst_v,
                               const int64_t* block_mapping, int64_t num_pairs, int64_t num_layers,
                               int64_t src_blocks, int64_t dst_blocks, int64_t block_bytes,
                               const musa_aiter_hip_claims* claims, void* stream);

/* ---- Paged-A [NB,NH,HD,BS] <-> linear [T,NH,HD] -------------------------------------------------
 * binding kv_transfer.py:350-376 (gather), :410-436 (scatter), :480-508 / :542-570 (multi-layer),
 * :615-639 / :671-695 / :741-767 / :799-825 (merged), :872-898 / :933-959 (MLA split);
 * replaces kv_transfer_float.mu:58-86, :169-235, :237-385, :387-671, :673-825, :1523-1590 and
 * lmcache_kv_transfer_extended.mu:577-628. */
#define MUSA_AITER_KV_HIP_PAGED_DECLS(SUFFIX)                                                                       \
  int musa_aiter_kv_paged_to_linear_##SUFFIX(const void* key_cache, const void* value_cache,                       \
                                             const int64_t* slot_mapping, void* out_k, void* out_v,                \
                                             int64_t num_tokens, int64_t num_blocks, int64_t num_heads,            \
                                             int64_t head_dim, int64_t block_size, void* stream);                  \
  int musa_aiter_kv_linear_to_paged_##SUFFIX(const void* key_linear, const void* value_linear,                     \
                                             const int64_t* slot_mapping, void* key_cache, void* value_cache,      \
                                             int64_t num_tokens, int64_t num_blocks, int64_t num_heads,            \
                                             int64_t head_dim, int64_t block_size, void* stream);                  \
  int musa_aiter_kv_paged_to_linear_multi_layer_##SUFFIX(                                                          \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, void* out_k, void* out_v,       \
      int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t num_heads, int64_t head_dim,             \
      int64_t block_size, void* stream);                                                                           \
  int musa_aiter_kv_linear_to_paged_multi_layer_##SUFFIX(                                                          \
      const void* key_linear, const void* value_linear, const int64_t* slot_mapping, void* key_cache,              \
      void* value_cache, int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,            \
      int64_t head_dim, int64_t block_size, void* stream);                                                         \
  int musa_aiter_kv_paged_to_merged_linear_##SUFFIX(const void* key_cache, const void* value_cache,                \
                                                    const int64_t* slot_mapping, void* out, int64_t num_tokens,    \
                                                    int64_t num_blocks, int64_t num_heads, int64_t head_dim,       \
                                                    int64_t block_size, void* stream);                             \
  int musa_aiter_kv_merged_linear_to_paged_##SUFFIX(const void* merged, const int64_t* slot_mapping,               \
                                                    void* key_cache, void* value_cache, int64_t num_tokens,        \
                                                    int64_t num_blocks, int64_t num_heads, int64_t head_dim,       \
                                                    int64_t block_size, void* stream);                             \
  int musa_aiter_kv_paged_to_merged_linear_multi_layer_##SUFFIX(                                                   \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, void* out, int64_t num_layers,  \
      int64_t num_tokens, int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size,             \
      void* stream);                                                                                               \
  int musa_aiter_kv_merged_linear_to_paged_multi_layer_##SUFFIX(                                                   \
      const void* merged, const int64_t* slot_mapping, void* key_cache, void* value_cache, int64_t num_layers,     \
      int64_t num_tokens, int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size,             \
      void* stream);                                                                                               \
  int musa_aiter_kv_paged_to_mla_linear_##SUFFIX(const void* kv_cache, const void* pe_cache,                      \
                                                 const int64_t* slot_mapping, void* out_kv, void* out_pe,          \
                                                 int64_t num_tokens, int64_t num_blocks, int64_t block_size,       \
                                                 int64_t kv_dim, int64_t pe_dim, void* stream);                    \
  int musa_aiter_kv_mla_linear_to_paged_##SUFFIX(const void* kv_linear, const void* pe_linear,                    \
                                                 const int64_t* slot_mapping, void* kv_cache, void* pe_cache,      \
                                                 int64_t num_tokens, int64_t num_blocks, int64_t block_size,       \
                                                 int64_t kv_dim, int64_t pe_dim, void* stream);

MUSA_AITER_KV_HIP_PAGED_DECLS(float)
MUSA_AITER_KV_HIP_PAGED_DECLS(half)
MUSA_AITER_KV_HIP_PAGED_DECLS(bfloat16)

/* ---- Dense preload for attention: block tables / CSR indices -> dense [B, S, NH, HD] --------------
 * load_and_reshape_flash: binding kv_transfer.py:1369-1440, replaces kv_transfer_float.mu:985-1076
 *   and :1420-1474; positions >= seq_lens[b] and invalid block ids are written as zeros.
 * reshape_and_cache_back_flash: binding kv_transfer.py:1443-1524, replaces
 *   kv_transfer_float.mu:1078-1164 and :1476-1521; the reverse scatter (duplicate destinations:
 *   the last (batch, position) in row-major order wins, like the reference's Python loop).
 * triton_indexed_to_dense: binding kv_transfer.py:1220-1288, replaces kv_transfer_float.mu:88-167
 *   and :1208-1254 (wrappers :1564-1587); caches are token-major [num_tokens, NH, HD]; dense
 *   token (b, pos) copies row kv_indices[kv_indptr[b] + pos] when that offset lies inside
 *   [kv_indptr[b], kv_indptr[b + 1]) and [0, index_count) and the row inside [0, num_tokens);
 *   other rows are zeros. */
#define MUSA_AITER_KV_HIP_DENSE_DECLS(SUFFIX)                                                                       \
  int musa_aiter_kv_load_and_reshape_flash_##SUFFIX(                                                               \
      const void* key_cache, const void* value_cache, const int64_t* block_tables, const int64_t* seq_lens,        \
      void* out_k, void* out_v, int64_t batch, int64_t dense_len, int64_t max_blocks, int64_t num_blocks,          \
      int64_t num_heads, int64_t head_dim, int64_t block_size, void* stream);                                      \
  int musa_aiter_kv_reshape_and_cache_back_flash_##SUFFIX(                                                         \
      const void* dense_k, const void* dense_v, const int64_t* block_tables, const int64_t* seq_lens,              \
      void* key_cache, void* value_cache, int64_t batch, int64_t dense_len, int64_t max_blocks,                    \
      int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size, void* stream);                  \
  int musa_aiter_kv_triton_indexed_to_dense_##SUFFIX(                                                              \
      const void* key_cache, const void* value_cache, const int64_t* kv_indptr, const int64_t* kv_indices,         \
      void* out_k, void* out_v, int64_t batch, int64_t dense_len, int64_t index_count, int64_t num_tokens,         \
      int64_t num_heads, int64_t head_dim, void* stream);

MUSA_AITER_KV_HIP_DENSE_DECLS(float)
MUSA_AITER_KV_HIP_DENSE_DECLS(half)
MUSA_AITER_KV_HIP_DENSE_DECLS(bfloat16)

/* ---- Paged block copies between same-layout caches [NB,NH,HD,BS] or [NL,NB,NH,HD,BS] -------------
 * binding kv_transfer.py:1962-2032 (float/half/bfloat16) and :1798-1868 (FP8 bytes, "_fp8_vec8");
 * replaces kv_transfer_float.mu:907-983, :1379-1418 (wrappers :1556-1563) and
 * fp8_kv_cache.mu:1462-1527.  block_mapping is a device int64 [num_pairs, 2] array of
 * (source, destination) block ids; a pair with a negative or out-of-range id is skipped and a
 * destination named by several pairs keeps the last pair.  Source and destination blocks of one
 * call must not overlap (the copy of all pairs runs concurrently). */
#define MUSA_AITER_KV_HIP_BLOCKS_DECL(NAME)                                                                         \
  int NAME(const void* src_key_cache, const void* src_value_cache, void* dst_key_cache, void* dst_value_cache,     \
           const int64_t* block_mapping, int64_t num_pairs, int64_t num_layers, int64_t src_blocks,                \
           int64_t dst_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size, void* stream);

MUSA_AITER_KV_HIP_BLOCKS_DECL(musa_aiter_kv_copy_paged_blocks_float)
MUSA_AITER_KV_HIP_BLOCKS_DECL(musa_aiter_kv_copy_paged_blocks_half)
MUSA_AITER_KV_HIP_BLOCKS_DECL(musa_aiter_kv_copy_paged_blocks_bfloat16)
MUSA_AITER_KV_HIP_BLOCKS_DECL(musa_aiter_kv_copy_paged_blocks_fp8_vec8)

/* ---- FP8 quant-store / dequant-gather (uint8 paged-A caches) ----------------------------------
 * binding kv_transfer.py:2401-2480 (vec4 scatter), :2485-2555 (scalar scatter), :2560-2640 (hd/bs
 * gathers), :2640-2800 (vec4 / scalar gathers), :2805-2980 (multi-layer); replaces
 * fp8_kv_cache.mu:146-272, :326-452, :454-740, :742-882, :884-1302, :1304-1460.
 * dtype_code: 1 float16, 2 bfloat16 (reference codes), 3 float32 (extension).
 * Scales are device float32: scalar (scale_mode 0), [NH] (1) or [NL, NH] (2).
 * Encoding follows the reference PyTorch encoder (kv_transfer.py:2161-2183) bit-exactly. */
#define MUSA_AITER_KV_HIP_FP8_DECLS(FMT)                                                                            \
  int musa_aiter_kv_linear_to_paged_fp8_##FMT(const void* key_linear, const void* value_linear,                    \
                                              const int64_t* slot_mapping, void* key_cache, void* value_cache,     \
                                              const float* k_scale, const float* v_scale, int64_t num_tokens,      \
                                              int64_t num_blocks, int64_t num_heads, int64_t head_dim,             \
                                              int64_t block_size, int dtype_code, void* stream);                   \
  int musa_aiter_kv_linear_to_paged_fp8_vec4_##FMT(                                                                \
      const void* key_linear, const void* value_linear, const int64_t* slot_mapping, void* key_cache,              \
      void* value_cache, const float* k_scale, const float* v_scale, int64_t num_tokens, int64_t num_blocks,       \
      int64_t num_heads, int64_t head_dim, int64_t block_size, int dtype_code, void* stream, int scale_mode);      \
  int musa_aiter_kv_paged_fp8_to_linear_##FMT(const void* key_cache, const void* value_cache,                      \
                                              const int64_t* slot_mapping, const float* k_scale,                   \
                                              const float* v_scale, void* out_k, void* out_v, int64_t num_tokens,  \
                                              int64_t num_blocks, int64_t num_heads, int64_t head_dim,             \
                                              int64_t block_size, int dtype_code, void* stream);                   \
  int musa_aiter_kv_paged_fp8_to_linear_vec4_##FMT(                                                                \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, const float* k_scale,           \
      const float* v_scale, void* out_k, void* out_v, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,   \
      int64_t head_dim, int64_t block_size, int dtype_code, void* stream, int scale_mode);                         \
  int musa_aiter_kv_linear_to_paged_fp8_multi_layer_##FMT(                                                         \
      const void* key_linear, const void* value_linear, const int64_t* slot_mapping, void* key_cache,              \
      void* value_cache, const float* k_scale, const float* v_scale, int64_t num_layers, int64_t num_tokens,       \
      int64_t num_blocks, int64_t num_heads, int64_t head_dim, int64_t block_size, int dtype_code, void* stream,   \
      int scale_mode);                                                                                             \
  int musa_aiter_kv_paged_fp8_to_linear_multi_layer_##FMT(                                                         \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, const float* k_scale,           \
      const float* v_scale, void* out_k, void* out_v, int64_t num_layers, int64_t num_tokens, int64_t num_blocks,  \
      int64_t num_heads, int64_t head_dim, int64_t block_size, int dtype_code, void* stream, int scale_mode);      \
  int musa_aiter_kv_paged_fp8_to_linear_hd64_bs16_##FMT(                                                           \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, const float* k_scale,           \
      const float* v_scale, void* out_k, void* out_v, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,   \
      int dtype_code, void* stream);                                                                               \
  int musa_aiter_kv_paged_fp8_to_linear_hd128_bs16_##FMT(                                                          \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, const float* k_scale,           \
      const float* v_scale, void* out_k, void* out_v, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,   \
      int dtype_code, void* stream);                                                                               \
  int musa_aiter_kv_paged_fp8_to_linear_hd128_bs32_##FMT(                                                          \
      const void* key_cache, const void* value_cache, const int64_t* slot_mapping, const float* k_scale,           \
      const float* v_scale, void* out_k, void* out_v, int64_t num_tokens, int64_t num_blocks, int64_t num_heads,   \
      int dtype_code, void* stream);

MUSA_AITER_KV_HIP_FP8_DECLS(e4m3)
MUSA_AITER_KV_HIP_FP8_DECLS(e5m2)

/* ---- LMCache legacy 6-D [NL,2,NB,BS,NH,HS] and MLA [NL,NB,BS,HS] <-> buffers -------------------
 * binding lmcache_kv_transfer.py:628-696 (_call_non_mla_symbol / _call_mla_symbol);
 * replaces kv_transfer_float.mu:1592-2030.  No-suffix = fp32, _u16 = 16-bit payloads. */
int lmcache_kv_buffer_to_paged(const void* kv_buffer, void* paged_kv_cache, const int64_t* slot_mapping,
                               int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t block_size,
                               int64_t num_heads, int64_t head_size, void* stream);
int lmcache_paged_to_kv_buffer(const void* paged_kv_cache, void* kv_buffer, const int64_t* slot_mapping,
                               int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t block_size,
                               int64_t num_heads, int64_t head_size, void* stream);
int lmcache_kv_buffer_to_paged_u16(const void* kv_buffer, void* paged_kv_cache, const int64_t* slot_mapping,
                                   int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t block_size,
                                   int64_t num_heads, int64_t head_size, void* stream);
int lmcache_paged_to_kv_buffer_u16(const void* paged_kv_cache, void* kv_buffer, const int64_t* slot_mapping,
                                   int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t block_size,
                                   int64_t num_heads, int64_t head_size, void* stream);
int lmcache_kv_buffer_to_paged_mla(const void* kv_buffer, void* paged_kv_cache, const int64_t* slot_mapping,
                                   int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t block_size,
                                   int64_t hidden_size, void* stream);
int lmcache_paged_to_kv_buffer_mla(const void* paged_kv_cache, void* kv_buffer, const int64_t* slot_mapping,
                                   int64_t num_layers, int64_t num_tokens, int64_t num_blocks, int64_t block_size,
                                   int64_t hidden_size, void* stream);
int lmcache_kv_buffer_to_paged_mla_u16(const void* kv_buffer, void* paged_kv_cache, const int64_t* slot_mapping,
                                       int64_t num_layers, int64_t num_tokens, int64_t num_blocks,
                                       int64_t block_size, int64_t hidden_size, void* stream);
int lmcache_paged_to_kv_buffer_mla_u16(const void* paged_kv_cache, void* kv_buffer, const int64_t* slot_mapping,
                                       int64_t num_layers, int64_t num_tokens, int64_t num_blocks,
                                       int64_t block_size, int64_t hidden_size, void* stream);

/* ---- LMCache SGLang-MP 2 x NL x [NB,BS,NH,HS] <-> [2,NL,M,NH*HS] --------------------------------
 * per-(axis, layer) plane: binding lmcache_kv_transfer.py:713-761 (_call_two_x_nl_symbol), replaces
 * kv_transfer_float.mu:2158-2308 and lmcache_kv_transfer_extended.mu:517-539;
 * all planes in one launch (cache_ptrs: host array of 2*NL device pointers, K layers then V
 * layers): replaces kv_transfer_float.mu:2072-2156 (coalesced u16). */
int lmcache_kv_buffer_to_paged_two_x_nl_float(const void* memory_tensor, void* cache, const int64_t* slot_mapping,
                                              int64_t kv_axis, int64_t layer_index, int64_t num_layers,
                                              int64_t memory_tokens, int64_t num_tokens,
                                              int64_t skip_prefix_n_tokens, int64_t num_blocks, int64_t block_size,
                                              int64_t num_heads, int64_t head_size, void* stream);
int lmcache_paged_to_kv_buffer_two_x_nl_float(void* memory_tensor, const void* cache, const int64_t* slot_mapping,
                                              int64_t kv_axis, int64_t layer_index, int64_t num_layers,
                                              int64_t memory_tokens, int64_t num_tokens,
                                              int64_t skip_prefix_n_tokens, int64_t num_blocks, int64_t block_size,
                                              int64_t num_heads, int64_t head_size, void* stream);
int lmcache_kv_buffer_to_paged_two_x_nl_u16(const void* memory_tensor, void* cache, const int64_t* slot_mapping,
                                            int64_t kv_axis, int64_t layer_index, int64_t num_layers,
                                            int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix_n_tokens,
                                            int64_t num_blocks, int64_t block_size, int64_t num_heads,
                                            int64_t head_size, void* stream);
int lmcache_paged_to_kv_buffer_two_x_nl_u16(void* memory_tensor, const void* cache, const int64_t* slot_mapping,
                                            int64_t kv_axis, int64_t layer_index, int64_t num_layers,
                                            int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix_n_tokens,
                                            int64_t num_blocks, int64_t block_size, int64_t num_heads,
                                            int64_t head_size, void* stream);
int lmcache_kv_buffer_to_paged_two_x_nl_coalesced_u16(const void* memory_tensor, const uint64_t* cache_ptrs,
                                                      const int64_t* slot_mapping, int64_t num_layers,
                                                      int64_t memory_tokens, int64_t num_tokens,
                                                      int64_t skip_prefix_n_tokens, int64_t num_blocks,
                                                      int64_t block_size, int64_t num_heads, int64_t head_size,
                                                      void* stream);
int lmcache_paged_to_kv_buffer_two_x_nl_coalesced_u16(void* memory_tensor, const uint64_t* cache_ptrs,
                                                      const int64_t* slot_mapping, int64_t num_layers,
                                                      int64_t memory_tokens, int64_t num_tokens, int64_t num_blocks,
                                                      int64_t block_size, int64_t num_heads, int64_t head_size,
                                                      void* stream);

/* ---- LMCache per-layer list caches [2,NB,BS,NH,HS] (binding lmcache_kv_transfer.py:874-993;
 * replaces kv_transfer_float.mu:2310-2600, lmcache_kv_transfer_extended.mu:495-515) ---- */
int lmcache_kv_buffer_to_paged_list_float(const void* memory_tensor, void* kvcache, const int64_t* slot_mapping,
                                          int64_t layer_index, int64_t num_layers, int64_t memory_tokens,
                                          int64_t num_tokens, int64_t skip_prefix, int64_t num_blocks,
                                          int64_t block_size, int64_t num_heads, int64_t head_size, void* stream);
int lmcache_paged_to_kv_buffer_list_float(void* memory_tensor, const void* kvcache, const int64_t* slot_mapping,
                                          int64_t layer_index, int64_t num_layers, int64_t memory_tokens,
                                          int64_t num_tokens, int64_t skip_prefix, int64_t num_blocks,
                                          int64_t block_size, int64_t num_heads, int64_t head_size, void* stream);
int lmcache_kv_buffer_to_paged_list_u16(const void* memory_tensor, void* kvcache, const int64_t* slot_mapping,
                                        int64_t layer_index, int64_t num_layers, int64_t memory_tokens,
                                        int64_t num_tokens, int64_t skip_prefix, int64_t num_blocks,
                                        int64_t block_size, int64_t num_heads, int64_t head_size, void* stream);
int lmcache_paged_to_kv_buffer_list_u16(void* memory_tensor, const void* kvcache, const int64_t* slot_mapping,
                                        int64_t layer_index, int64_t num_layers, int64_t memory_tokens,
                                        int64_t num_tokens, int64_t skip_prefix, int64_t num_blocks,
                                        int64_t block_size, int64_t num_heads, int64_t head_size, void* stream);
int lmcache_kv_buffer_to_paged_list2_u16(const void* memory_tensor, void* kvcache0, void* kvcache1,
                                         const int64_t* slot_mapping, int64_t memory_tokens, int64_t num_tokens,
                                         int64_t skip_prefix, int64_t num_blocks, int64_t block_size,
                                         int64_t num_heads, int64_t head_size, void* stream);
int lmcache_paged_to_kv_buffer_list2_u16(void* memory_tensor, const void* kvcache0, const void* kvcache1,
                                         const int64_t* slot_mapping, int64_t memory_tokens, int64_t num_tokens,
                                         int64_t skip_prefix, int64_t num_blocks, int64_t block_size,
                                         int64_t num_heads, int64_t head_size, void* stream);
/* The reference extension's kernel variants of the list2 transfer (lmcache_kv_transfer_ext.cpp:42-125:
 * _coalesced, _contiguous, _contiguous_bulk, _torchmusa_style, _sorted), which it selects by environment
 * variable and which all move the same bytes: here each is the list2 entry above, with the same
 * arguments (the _sorted gather's sort order of the slots is accepted and not needed). */
int lmcache_kv_buffer_to_paged_list2_u16_coalesced(const void* memory_tensor, void* kvcache0, void* kvcache1,
                                                   const int64_t* slot_mapping, int64_t memory_tokens,
                                                   int64_t num_tokens, int64_t skip_prefix, int64_t num_blocks,
                                                   int64_t block_size, int64_t num_heads, int64_t head_size,
                                                   void* stream);
#define MUSA_AITER_KV_HIP_LIST2_GATHER_VARIANT(VARIANT)                                                           \
  int lmcache_paged_to_kv_buffer_list2_u16_##VARIANT(void* memory_tensor, const void* kvcache0,                  \
                                                     const void* kvcache1, const int64_t* slot_mapping,           \
                                                     int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix, \
                                                     int64_t num_blocks, int64_t block_size, int64_t num_heads,   \
                                                     int64_t head_size, void* stream);
MUSA_AITER_KV_HIP_LIST2_GATHER_VARIANT(coalesced)
MUSA_AITER_KV_HIP_LIST2_GATHER_VARIANT(contiguous)
MUSA_AITER_KV_HIP_LIST2_GATHER_VARIANT(contiguous_bulk)
MUSA_AITER_KV_HIP_LIST2_GATHER_VARIANT(torchmusa_style)
#undef MUSA_AITER_KV_HIP_LIST2_GATHER_VARIANT
int lmcache_paged_to_kv_buffer_list2_u16_sorted(void* memory_tensor, const void* kvcache0, const void* kvcache1,
                                                const int64_t* slot_mapping, const uint8_t* sorted_indices_bytes,
                                                int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix,
                                                int64_t num_blocks, int64_t block_size, int64_t num_heads,
                                                int64_t head_size, void* stream);

/* ---- LMCache MLA per-layer lists [NB,BS,HS] <-> [1,NL,M,HS] (binding lmcache_kv_transfer.py:920-950;
 * replaces lmcache_kv_transfer_extended.mu:541-575) ---- */
#define MUSA_AITER_KV_HIP_MLA_LIST_DECLS(SUFFIX)                                                                    \
  int lmcache_mla_buffer_to_paged_list_##SUFFIX(const void* memory_tensor, void* kvcache,                          \
                                                const int64_t* slot_mapping, int64_t layer_index,                  \
                                                int64_t memory_tokens, int64_t num_tokens, int64_t skip_prefix,    \
                                                int64_t num_blocks, int64_t block_size, int64_t head_size,         \
                                                void* stream);                                                     \
  int lmcache_mla_paged_to_buffer_list_##SUFFIX(void* memory_tensor, const void* kvcache,                          \
                                                const int64_t* slot_mapping, int64_t layer_index,                  \
                                                int64_t memory_tokens, int64_t num_tokens, int64_t num_blocks,     \
                                                int64_t block_size, int64_t head_size, void* stream);

MUSA_AITER_KV_HIP_MLA_LIST_DECLS(float)
MUSA_AITER_KV_HIP_MLA_LIST_DECLS(half)
MUSA_AITER_KV_HIP_MLA_LIST_DECLS(bfloat16)
MUSA_AITER_KV_HIP_MLA_LIST_DECLS(u16)

/* ---- DSV4 opaque byte rows (binding kv_transfer.py:4209-4253, :4310-4406;
 * replaces kv_transfer_float.mu:3088-3275).  Out-of-range rows are skipped.
 * The layer-table entry takes device arrays of per-layer base addresses. ---- */
int musa_aiter_kv_copy_paged_rows_u8(const void* src, void* dst, const int64_t* src_indices,
                                     const int64_t* dst_indices, int64_t num_rows, int64_t item_bytes,
                                     int64_t src_num_rows, int64_t dst_num_rows, void* stream);
int musa_aiter_kv_copy_paged_rows_layer_table_u8(const uint64_t* src_ptr_table, const uint64_t* dst_ptr_table,
                                                 const int64_t* src_indices, const int64_t* dst_indices,
                                                 int64_t num_rows, int64_t item_bytes, int64_t num_layers,
                                                 int64_t src_num_rows, int64_t dst_num_rows, void* stream);
int musa_aiter_kv_copy_paged_rows_contig_layers_u8(const void* src_base, void* dst_base, const int64_t* src_indices,
                                                   const int64_t* dst_indices, int64_t num_rows, int64_t item_bytes,
                                                   int64_t num_layers, int64_t src_num_rows, int64_t dst_num_rows,
                                                   void* stream);

/* ---- LMCache DSV4 strided block transfer (binding lmcache_kv_transfer.py:1355-1400;
 * replaces kv_transfer_float.mu:3302-3405).  paged_ptrs: host array of num_layers (<= 128)
 * device page bases; direction 0 staging->pages, 1 pages->staging; mode 0 plain rows,
 * mode 1 values block then scales block (value_bytes + scale_bytes == row_bytes). ---- */
int lmcache_kv_strided_block_transfer(void* staging, const uint64_t* paged_ptrs, const int64_t* block_ids,
                                      int64_t direction, int64_t num_layers, int64_t idx_start, int64_t n_valid,
                                      int64_t offset_in_object, int64_t staging_tokens, int64_t block_size,
                                      int64_t row_bytes, int64_t paged_block_stride, int64_t mode,
                                      int64_t value_bytes, int64_t scale_bytes, void* stream);

/* ---- SGLang HiCache layer-first / page-first transfers (binding hicache_transfer.py:59-82,
 * :190-258; replaces hicache_transfer.mu:4-98).  For each item whose two page indices are both
 * non-negative and each layer in [start_layer, start_layer + num_layers), item_size_bytes
 * (rounded down to whole 64-bit words) move from src + page * src_page_stride + layer *
 * src_layer_stride to the matching destination offset, for K and, when both V pointers are
 * non-null, for V.  Indices are int64 device arrays and are not range-checked; a destination
 * page named by several items receives one of them (the Python layer validates indices and
 * keeps the last item through musa_aiter_hip_copy_rows_paged). ---- */
int musa_aiter_hicache_transfer_abi_version(void);
int musa_aiter_hicache_transfer_bytes(const void* src_k, void* dst_k, const void* src_v, void* dst_v,
                                      const int64_t* src_indices, const int64_t* dst_indices, int64_t num_items,
                                      int64_t start_layer, int64_t num_layers, int64_t item_size_bytes,
                                      int64_t src_page_stride_bytes, int64_t src_layer_stride_bytes,
                                      int64_t dst_page_stride_bytes, int64_t dst_layer_stride_bytes, void* stream);

/* ---- LMCache host <-> device batch copies (binding lmcache_musa_batch_copy.py:121-215 through
 * the extension object of lmcache_musa_batch_copy_ext.py:19-43; replaces
 * lmcache_musa_batch_copy_ext.cpp:41-277, which wraps musaMemcpyBatchAsync / musaMemcpyAsync).
 * Copies count byte ranges srcs[i] -> dsts[i] (sizes[i] bytes), all host -> device (direction 0)
 * or all device -> host (direction 1), on `stream`.  mode 0: a range whose host side is pinned host
 * memory mapped for the device goes through one batch-copy kernel launch per 96 ranges on at most
 * 64 workgroups; mode 1 (the reference's prefer_overlap_with_compute hint): the same kernel on at
 * most 16 workgroups, leaving the other compute units to concurrent kernels; pageable
 * ranges in modes 0 and 1, and every range in mode 2 (the reference's execute_copy_loop), go through
 * hipMemcpyAsync.  Destination ranges must not overlap.  The version probe returns
 * hipRuntimeGetVersion / hipDriverGetVersion. ---- */
int musa_aiter_hip_batch_copy_abi_version(void);
int musa_aiter_hip_runtime_versions(int* runtime_version, int* driver_version);
int musa_aiter_hip_batch_copy(void* const* dsts, const void* const* srcs, const uint64_t* sizes, int64_t count,
                              int direction, int mode, void* stream);

/* ---- CacheGen-style uniform-bin codec (binding kv_transfer.py:1048-1108; replaces
 * kv_transfer_float.mu:828-898).  The two reference entries keep the reference kernels'
 * contracts: encode_float writes bin = clamp(trunc(fma(x - min_val, scale, 0.5f)), 0,
 * num_bins - 1) for `numel` float32 elements (num_bins in [1, 256]); decode_float writes
 * output[i] = codebook[encoded[i]] reading the float32 codebook from global memory, so every
 * code must be inside the caller's codebook.
 *
 * musa_aiter_hip_cachegen_encode is the whole of kv_transfer.py:1111-1172 on the device, with no
 * host synchronisation: input_dtype 0 float32, 1 float16, 2 bfloat16, 3 float64 (widened or
 * rounded to float32 first), num_bins in [2, 256]; encoded[numel] uint8, codebook[num_bins] and
 * cdf[num_bins + 1] float32 are written; `workspace` is device memory of at least
 * musa_aiter_hip_cachegen_workspace_bytes() bytes, private to the call until it completes.
 * native_rounding = 1 (float32 only) selects the reference kernel's rounding above, 0 the torch
 * path's: bin = clamp(rint((x - min) * ((1 / (max - min)) * (num_bins - 1))), 0, num_bins - 1).
 * musa_aiter_hip_cachegen_decode gathers entries of elem_bytes (1, 2, 4, 8 or 16; `table`
 * aligned to it) from a table of table_len entries (1..256); with table_len < 256 the caller
 * clears *max_code (device int32) beforehand and afterwards finds there the largest code at or
 * past table_len, or 0 when every code was inside the table. ---- */
int musa_aiter_kv_cachegen_encode_float(const void* input, void* encoded, float min_val, float scale, int64_t numel,
                                        int64_t num_bins, void* stream);
int musa_aiter_kv_cachegen_decode_float(const void* encoded, const void* codebook, void* output, int64_t numel,
                                        void* stream);
int64_t musa_aiter_hip_cachegen_workspace_bytes(void);
int musa_aiter_hip_cachegen_encode(const void* input, int input_dtype, int64_t numel, int64_t num_bins,
                                   int native_rounding, void* encoded, void* codebook, void* cdf, void* workspace,
                                   int64_t workspace_bytes, void* stream);
int musa_aiter_hip_cachegen_decode(const void* encoded, int64_t numel, const void* table, int64_t table_len,
                                   int elem_bytes, void* output, int32_t* max_code, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MUSA_AITER_KV_HIP_H_ */
