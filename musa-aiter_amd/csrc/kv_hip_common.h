// Shared device helpers for the MI355X (gfx950) KV-cache movement kernels.
//
// Everything here is written for CDNA4 wave64 execution: 64-lane ballots,
// 16-byte global_load/store_dwordx4 payload moves and scalar (wave-uniform)
// slot resolution.  No MFMA is used: the path is a bandwidth-bound copy.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvhip {

constexpr int kWave = 64;
constexpr int kWavesPerBlock = 4;
constexpr int kBlockThreads = kWave * kWavesPerBlock;

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));
using u32x2 = uint32_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// Vector memory helpers.  Two cache policies:
//  * stream (non-temporal): for accesses whose wave instruction covers whole
//    cache lines (coalesced token rows); the data is touched exactly once.
//  * cached: for strided accesses where one instruction touches many lines
//    partially and later instructions of the same wave finish those lines;
//    L2 must keep and merge them (write-combining for partial-line stores).
// ---------------------------------------------------------------------------
template <int VEC>
struct VecType;
template <>
struct VecType<16> { using T = u32x4; };
template <>
struct VecType<8> { using T = u32x2; };
template <>
struct VecType<4> { using T = uint32_t; };
template <>
struct VecType<2> { using T = uint16_t; };
template <>
struct VecType<1> { using T = uint8_t; };

// Every pointer these helpers see is device (global) memory, never LDS or
// scratch: the casts to address space 1 let the compiler emit global_load /
// global_store instead of flat accesses, which also count against lgkmcnt.
#define KVHIP_GLOBAL __attribute__((address_space(1)))

template <int VEC>
__device__ __forceinline__ typename VecType<VEC>::T ldv(const uint8_t* p) {
  using T = typename VecType<VEC>::T;
  return __builtin_nontemporal_load((const KVHIP_GLOBAL T*)(p));
}

template <int VEC>
__device__ __forceinline__ void stv(uint8_t* p, typename VecType<VEC>::T v) {
  using T = typename VecType<VEC>::T;
  __builtin_nontemporal_store(v, (KVHIP_GLOBAL T*)(p));
}

// Streaming 16-byte accesses (whole lines per wave instruction).
__device__ __forceinline__ u32x4 ld16(const uint8_t* p) { return ldv<16>(p); }
__device__ __forceinline__ void st16(uint8_t* p, u32x4 v) { stv<16>(p, v); }
// Cached 16-byte accesses (strided, partial lines per wave instruction).
__device__ __forceinline__ u32x4 ld16_cached(const uint8_t* p) { return *(const KVHIP_GLOBAL u32x4*)(p); }
__device__ __forceinline__ void st16_cached(uint8_t* p, u32x4 v) { *(KVHIP_GLOBAL u32x4*)(p) = v; }

// ---------------------------------------------------------------------------
// Raw buffer accesses (gfx9-family descriptor, stride 0).  The descriptor
// covers 2 GiB from a wave-uniform base; a lane that passes kOffOob as its
// offset turns its access into a hardware no-op (loads return zero, stores
// are dropped), so masked lanes need no branch.  Keeping the memory
// instructions unconditional lets the compiler count outstanding loads
// exactly, which keeps a prefetched load in flight across LDS barriers.
// ---------------------------------------------------------------------------
using buf_t = __amdgpu_buffer_rsrc_t;
constexpr uint32_t kOffOob = 0x80000000u;
constexpr int kBufNT = 2;  // cache policy bits: non-temporal
// Non-temporal and agent scope (sc1): the store writes through the L2 of the
// XCD that issues it.  Each of MI355X's eight XCDs has its own L2, so a kernel
// ends by writing its dirty L2 lines back; stores that wrote through leave
// none.  Measured on sequentially written outputs: a 61 MB gather 13.0 ->
// 12.1 us, a 67 MB 2 x NL chunk 13.0 -> 12.6 us, the 34 GB cfg 2 gather
// +1.1 %.  Used only for destination rows of whole 128-byte lines (656-byte
// rows written through were 7 % slower: their shared lines left the L2 once
// per row); the tile scatter's random blocks and the dense preload's gathers
// were no faster with it and keep kBufNT.
constexpr int kBufWT = kBufNT | 16;

__device__ __forceinline__ buf_t make_buf(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0x7FFFFFFF, 0x00020000);
}
__device__ __forceinline__ u32x4 buf_ld16(buf_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kBufNT);
}
// Per-lane offset `off` plus a wave-uniform offset `soff` (an SGPR operand).
__device__ __forceinline__ u32x4 buf_ld16(buf_t r, uint32_t off, uint32_t soff) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, kBufNT);
}
// Cached (default policy) load, for wave instructions that touch lines
// partially and leave the rest of each line to later instructions.
__device__ __forceinline__ u32x4 buf_ld16_cached(buf_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ void buf_st16(buf_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kBufNT);
}
// The same store with cache-policy bits CP (kBufNT or kBufWT).
template <int CP>
__device__ __forceinline__ void buf_st16_p(buf_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, CP);
}
template <int ELT>
__device__ __forceinline__ void buf_st_elem(buf_t r, uint32_t off, uint32_t v) {
  if constexpr (ELT == 1) __builtin_amdgcn_raw_buffer_store_b8(static_cast<uint8_t>(v), r, off, 0, 0);
  else if constexpr (ELT == 2) __builtin_amdgcn_raw_buffer_store_b16(static_cast<uint16_t>(v), r, off, 0, 0);
  else __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, 0);
}

// ---------------------------------------------------------------------------
// XCD-aware workgroup order.  MI355X dispatches workgroup i of a launch (in
// linearised grid order) to XCD i mod 8, and each XCD has its own L2.  With
// ON, a workgroup takes the coordinates of position w of the grid, where XCD
// k's workgroups cover one contiguous eighth of the grid in order: tiles that
// neighbour each other (overlapping slot windows, the row groups of one
// cache block) then run on the same XCD.  The grid must hold fewer than 2^32
// workgroups.
// ---------------------------------------------------------------------------
struct WgXyz {
  uint32_t x, y, z;
};

template <bool ON>
__device__ __forceinline__ WgXyz xcd_contiguous_wg() {
  if constexpr (!ON) {
    return {blockIdx.x, blockIdx.y, blockIdx.z};
  } else {
    constexpr uint32_t kXcds = 8;
    const uint32_t gx = gridDim.x, gy = gridDim.y;
    const uint32_t total = gx * gy * gridDim.z;
    const uint32_t lin = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const uint32_t xcd = lin % kXcds, idx = lin / kXcds;
    const uint32_t q = total / kXcds, r = total % kXcds;  // XCDs below r take q + 1 workgroups
    const uint32_t w = xcd < r ? xcd * (q + 1) + idx : r * (q + 1) + (xcd - r) * q + idx;
    const uint32_t gxy = gx * gy;
    const uint32_t z = w / gxy;
    const uint32_t rem = w - z * gxy;
    const uint32_t y = rem / gx;
    return {rem - y * gx, y, z};
  }
}

// ---------------------------------------------------------------------------
// Wave-level helpers (wave64).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x) & (kWave - 1); }

__device__ __forceinline__ int wave_in_block() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
}

__device__ __forceinline__ uint64_t ballot(bool pred) {
  return static_cast<uint64_t>(__ballot(pred));
}

__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane(static_cast<uint32_t>(v), lane);
  const uint32_t hi = __builtin_amdgcn_readlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32), lane);
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}

// Value of a 64-bit per-lane quantity held by lane (lane_id - 1); lane 0 gets its own.
__device__ __forceinline__ int64_t from_prev_lane(int64_t v) {
  return __shfl_up(static_cast<long long>(v), 1);
}

// ---------------------------------------------------------------------------
// Claim tags for last-writer-wins scatter.  A scatter that may see duplicate
// destination slots first records, per destination slot, the largest
// (epoch, token+1) pair among the tokens targeting it; only the token whose
// tag survives writes.  The epoch advances per call so the array never needs
// clearing between calls on one stream.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t claim_tag(uint32_t epoch, int64_t token) {
  return (static_cast<uint64_t>(epoch) << 32) | static_cast<uint64_t>(token + 1);
}

// ---------------------------------------------------------------------------
// Block-table addressing of a dense [batch, dense_len] token range (the
// Flash-style preload, reference csrc/kvcache/kv_transfer_float.mu:985-1037):
// token t = b * dense_len + pos lives in slot
//   block_tables[b, pos / block_size] * block_size + pos % block_size
// while pos < seq_lens[b], the logical block is below max_blocks and the block
// id lies in [0, num_blocks); otherwise it has no slot (-1).  The host keeps
// batch * dense_len, max_blocks and block_size below 2^31.
// ---------------------------------------------------------------------------
struct BlockTableSlots {
  const int64_t* block_tables;  // [batch, max_blocks]; nullptr: slots come from a vector
  const int64_t* seq_lens;      // [batch]
  int64_t num_blocks;
  uint32_t dense_len;
  int32_t max_blocks;
  int32_t block_size;
};

__device__ __forceinline__ int64_t block_table_slot(const BlockTableSlots& bt, int64_t t) {
  const uint32_t tt = static_cast<uint32_t>(t);
  const uint32_t b = tt / bt.dense_len;
  const int32_t pos = static_cast<int32_t>(tt - b * bt.dense_len);
  if (pos >= bt.seq_lens[b]) return -1;
  const int32_t lb = pos / bt.block_size;
  if (lb >= bt.max_blocks) return -1;
  const int64_t blk = bt.block_tables[static_cast<int64_t>(b) * bt.max_blocks + lb];
  if (blk < 0 || blk >= bt.num_blocks) return -1;
  return blk * bt.block_size + (pos - lb * bt.block_size);
}

// Row of dense token u = b * dense_len + pos in a CSR index table (SGLang's
// kv_indptr / kv_indices, reference csrc/kvcache/kv_transfer_float.mu:88-133):
// indices[indptr[b] + pos] when that offset lies inside both [indptr[b],
// indptr[b + 1]) and the index vector, else -1.
__device__ __forceinline__ int64_t csr_row(const int64_t* indptr, const int64_t* indices, uint32_t dense_len,
                                           int64_t index_count, int64_t u) {
  const uint32_t uu = static_cast<uint32_t>(u);
  const uint32_t b = uu / dense_len;
  const int64_t pos = static_cast<int64_t>(uu - b * dense_len);
  const int64_t start = indptr[b];
  const int64_t end = indptr[b + 1];
  const int64_t off = start + pos;
  if (start < 0 || end < start || off >= end || off >= index_count) return -1;
  return indices[off];
}

// ---------------------------------------------------------------------------
// 16-bit element access inside a 16-byte register vector.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t half_of(uint32_t w, int hi) { return hi ? (w >> 16) : (w & 0xFFFFu); }

__device__ __forceinline__ uint32_t elem16(const u32x4& v, int idx) {
  return half_of(v[idx >> 1], idx & 1);
}

__device__ __forceinline__ uint32_t elem8(const u32x4& v, int idx) {
  return (v[idx >> 2] >> (8 * (idx & 3))) & 0xFFu;
}

// Pack the 16-bit lanes `lo` (bits 0..15 used) and `hi` into one dword.
__device__ __forceinline__ uint32_t pack16(uint32_t lo, uint32_t hi) { return (lo & 0xFFFFu) | (hi << 16); }

// ---------------------------------------------------------------------------
// Floating-point conversions with the exact rounding torch uses on the CPU:
// bf16 and fp16 are produced round-to-nearest-even; widening is exact.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

__device__ __forceinline__ float f16_bits_to_f32(uint32_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(b));
  return static_cast<float>(h);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;  // canonical quiet NaN, as c10::BFloat16
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  // Keep the fp32 value opaque so the backend cannot fold a preceding fp32
  // multiply and this conversion into v_fma_mix with a +0.0 addend, which
  // would turn a -0.0 product into +0.0 (torch keeps the sign of zero).
  __asm__ volatile("" : "+v"(f));
  const _Float16 h = static_cast<_Float16>(f);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
}

// Linear-side element types for the FP8 codec paths.
enum LinDtype : int { kLinF32 = 0, kLinF16 = 1, kLinBF16 = 2 };

template <int LDT>
__device__ __forceinline__ float lin_to_f32(uint32_t bits) {
  if constexpr (LDT == kLinBF16) return bf16_bits_to_f32(bits);
  else if constexpr (LDT == kLinF16) return f16_bits_to_f32(bits);
  else return __uint_as_float(bits);
}

template <int LDT>
__device__ __forceinline__ uint32_t f32_to_lin(float f) {
  if constexpr (LDT == kLinBF16) return f32_to_bf16_bits(f);
  else if constexpr (LDT == kLinF16) return f32_to_f16_bits(f);
  else return __float_as_uint(f);
}

// ---------------------------------------------------------------------------
// FP8 codec with the reference's exact rules (musa_aiter/ops/kv_transfer.py
// :2161-2200, the PyTorch implementation, not its MUSA kernels):
//   * w = x / scale (IEEE fp32 division, round to nearest even);
//   * sign = (w < 0); non-finite w encodes as a signed-by-`w<0` zero;
//   * |w| is clamped to (2 - 2^-M) * 2^Emax  (E4M3 480, E5M2 114688);
//   * |w| below 2^(1-bias) flushes to a signed zero (no subnormals);
//   * the mantissa is rounded half-to-even, carrying into the exponent.
// Decoding maps exponent field 0 to a signed zero and every other code to
// (1 + m/2^M) * 2^(E-bias), including the all-ones patterns.
// ---------------------------------------------------------------------------
enum Codec : int { kCopy = 0, kE4M3 = 1, kE5M2 = 2 };

template <int CODEC>
struct Fp8Fmt;

template <>
struct Fp8Fmt<kE4M3> {
  static constexpr int kMant = 3;
  static constexpr uint32_t kMaxBits = 0x43F00000u;     // 480.0f
  static constexpr uint32_t kMinNormBits = 0x3C800000u; // 2^-6
  static constexpr int kShift = 23 - kMant;             // 20
  static constexpr uint32_t kExpOffset = 127 - 7;       // fp32 bias - fp8 bias
  static constexpr uint32_t kExpMask = 0x78u;
};

template <>
struct Fp8Fmt<kE5M2> {
  static constexpr int kMant = 2;
  static constexpr uint32_t kMaxBits = 0x47E00000u;     // 114688.0f
  static constexpr uint32_t kMinNormBits = 0x38800000u; // 2^-14
  static constexpr int kShift = 23 - kMant;             // 21
  static constexpr uint32_t kExpOffset = 127 - 15;
  static constexpr uint32_t kExpMask = 0x7Cu;
};

// Encode w (already the correctly rounded quotient x/scale) to an FP8 byte.
template <int CODEC>
__device__ __forceinline__ uint32_t fp8_encode(float w) {
  using F = Fp8Fmt<CODEC>;
  const uint32_t bits = __float_as_uint(w);
  const uint32_t sign = (w < 0.0f) ? 0x80u : 0u;
  uint32_t a = bits & 0x7FFFFFFFu;
  const bool normal = (a >= F::kMinNormBits) && (a < 0x7F800000u);
  a = a < F::kMaxBits ? a : F::kMaxBits;
  const uint32_t lsb = (a >> F::kShift) & 1u;
  // Round the fp32 mantissa to kMant bits (half to even) and re-bias the
  // exponent in one add: the carry out of the mantissa lands in the exponent.
  const uint32_t body =
      (a + ((1u << (F::kShift - 1)) - 1u) + lsb - (F::kExpOffset << 23)) >> F::kShift;
  return sign | (normal ? body : 0u);
}

template <int CODEC>
__device__ __forceinline__ float fp8_decode(uint32_t byte) {
  using F = Fp8Fmt<CODEC>;
  uint32_t bits = ((byte & 0x7Fu) << F::kShift) + (F::kExpOffset << 23);
  bits = (byte & F::kExpMask) ? bits : 0u;
  bits |= (byte & 0x80u) << 24;
  return __uint_as_float(bits);
}

// Division x / s rounded to nearest even, as torch's CPU `/` on float32.
// The default HIP compilation mode emits the correctly rounded
// v_div_scale/v_div_fmas/v_div_fixup sequence for this operator.
__device__ __forceinline__ float div_rn(float x, float s) { return x / s; }

// ---------------------------------------------------------------------------
// Quantiser quotient with a hoisted reciprocal.  For one scale s the lane
// computes r = RN(1/s) once (an exact division); per element
//   q0 = x*r,  q1 = q0 + RN(x - s*q0)*r,  q = q1 + RN(x - s*q1)*r
// (residuals exact through FMA) equals RN(x/s) whenever s and |x| lie in
// [2^-60, 2^60] (x = +-0 gives +0, which the encoder treats like -0): the
// first correction makes q1 faithful, the second is Markstein's final
// correction with a correctly rounded reciprocal.  No over- or underflow can
// occur in that range.  Elements outside it use div_rn.
//
// When x has at most 12 significant bits (every bf16 and fp16 value) q1 is
// already RN(x/s): checked exhaustively over every pair of significands (all
// 2^11 x all 2^23 for 12-bit x; tests/quotient_check.c), and both sides scale
// exactly by powers of two inside the range, so those inputs skip the second
// correction (2 of the ~13 VALU operations per quantised element).
// ---------------------------------------------------------------------------
constexpr uint32_t kFastLoBits = 0x21800000u;  // 2^-60
constexpr uint32_t kFastHiBits = 0x5D800000u;  // 2^60

__device__ __forceinline__ bool fast_scale_ok(float s) {
  return (__float_as_uint(s) - kFastLoBits) < (kFastHiBits - kFastLoBits);
}

// NARROW: x is a widened bf16 / fp16 value (at most 12 significant bits).
template <bool NARROW>
__device__ __forceinline__ float quot_fast(float x, float s, float r) {
  const float q0 = x * r;
  const float e0 = __builtin_fmaf(-s, q0, x);
  const float q1 = __builtin_fmaf(e0, r, q0);
  if constexpr (NARROW) return q1;
  const float e1 = __builtin_fmaf(-s, q1, x);
  return __builtin_fmaf(e1, r, q1);
}

// Encoder for a quotient known to be +0 or finite with 2^-120 <= |w| < 2^126
// (the fast range): the sign is the sign bit and no non-finite check is needed.
template <int CODEC>
__device__ __forceinline__ uint32_t fp8_encode_fast(float w) {
  using F = Fp8Fmt<CODEC>;
  const uint32_t bits = __float_as_uint(w);
  uint32_t a = bits & 0x7FFFFFFFu;
  const bool normal = a >= F::kMinNormBits;
  a = a < F::kMaxBits ? a : F::kMaxBits;
  const uint32_t lsb = (a >> F::kShift) & 1u;
  const uint32_t body =
      (a + ((1u << (F::kShift - 1)) - 1u) + lsb - (F::kExpOffset << 23)) >> F::kShift;
  return ((bits >> 24) & 0x80u) | (normal ? body : 0u);
}

// Hardware encoder for the fast range.  gfx950's v_cvt_pk_fp8_f32 /
// v_cvt_pk_bf8_f32 (OCP formats, round to nearest even, no saturation)
// produce the reference byte for every finite quotient once values below the
// smallest normal are flushed to a signed zero: checked exhaustively on the
// device over all finite fp32 inputs.  E4M3 matches everywhere (overflow
// gives 0x7F|sign, the reference's 480 clamp byte); E5M2 matches up to its
// largest normal 57344, above which the reference keeps exponent-31 codes and
// the callers must use fp8_encode_fast instead.
//
// The flush is w * step, step = clamp(|w| * 2^24 / m - (2^24 - 1), 0, 1) for the
// smallest normal m = 2^E: one fma (exact up to its single rounding; the
// product and the constant are exact) whose result is <= 0 exactly when
// |w| <= pred(m) = m - m * 2^-24 and >= 1 when |w| >= m, clamped by the
// instruction's clamp bit; w * +0 keeps w's sign.  Two VALU operations and no
// lane mask, where a compare and a select need three and a wait state.
// Checked against the compare-and-select form on every finite fp32 value.
template <int CODEC>
__device__ __forceinline__ float fp8_flush_small(float w) {
  constexpr float kBig = (CODEC == kE4M3) ? 0x1p30f : 0x1p38f;  // 2^24 / m
  const float t = __builtin_fmaf(__builtin_fabsf(w), kBig, -16777215.0f);
  return w * __builtin_amdgcn_fmed3f(t, 0.0f, 1.0f);
}

template <int CODEC>
constexpr uint32_t kHwEncodeMaxBits = (CODEC == kE4M3) ? 0x7F7FFFFFu : 0x47600000u;  // all finite / 57344

// Four quotients -> four bytes (element i in byte i).  FLUSH may be false
// when no quotient of the group lies below the smallest normal.
template <int CODEC, bool FLUSH = true>
__device__ __forceinline__ uint32_t fp8_pack4_hw(float w0, float w1, float w2, float w3) {
  if constexpr (FLUSH) {
    w0 = fp8_flush_small<CODEC>(w0);
    w1 = fp8_flush_small<CODEC>(w1);
    w2 = fp8_flush_small<CODEC>(w2);
    w3 = fp8_flush_small<CODEC>(w3);
  }
  int r;
  if constexpr (CODEC == kE4M3) {
    r = __builtin_amdgcn_cvt_pk_fp8_f32(w0, w1, 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(w2, w3, r, true);
  } else {
    r = __builtin_amdgcn_cvt_pk_bf8_f32(w0, w1, 0, false);
    r = __builtin_amdgcn_cvt_pk_bf8_f32(w2, w3, r, true);
  }
  return static_cast<uint32_t>(r);
}

// Magnitude range of a tile's linear inputs, tracked on the raw bits: the
// minimum of (|x| - 1) (so zeros drop out) and the maximum of |x|.  16-bit
// inputs are tracked two per dword with packed 16-bit integer min/max.
using u16x2 = unsigned short __attribute__((ext_vector_type(2)));

template <int LDT>
struct InputRange {
  static constexpr bool kWide = (LDT == kLinF32);
  uint32_t lo32 = 0xFFFFFFFFu;
  uint32_t hi32 = 0u;
  u16x2 lo16 = {0xFFFF, 0xFFFF};
  u16x2 hi16 = {0, 0};

  __device__ __forceinline__ void add(const u32x4& v) {
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      if constexpr (kWide) {
        const uint32_t a = v[w] & 0x7FFFFFFFu;
        lo32 = min(lo32, a - 1u);
        hi32 = max(hi32, a);
      } else {
        const u16x2 a = __builtin_bit_cast(u16x2, v[w] & 0x7FFF7FFFu);
        lo16 = __builtin_elementwise_min(lo16, a - u16x2{1, 1});
        hi16 = __builtin_elementwise_max(hi16, a);
      }
    }
  }

  __device__ __forceinline__ uint32_t lo() const {
    if constexpr (kWide) return lo32;
    else return lo16.x < lo16.y ? lo16.x : lo16.y;
  }
  __device__ __forceinline__ uint32_t hi() const {
    if constexpr (kWide) return hi32;
    else return hi16.x > hi16.y ? hi16.x : hi16.y;
  }

  // Smallest nonzero |x| of the tracked inputs (+inf bits when all are zero).
  __device__ __forceinline__ float min_abs_nonzero() const {
    const uint32_t m = lo() + 1u;  // wraps to 0 when every input was zero
    if constexpr (LDT == kLinF32) return m == 0u ? __uint_as_float(0x7F800000u) : __uint_as_float(m);
    else if constexpr (LDT == kLinBF16) return m > 0xFFFFu ? __uint_as_float(0x7F800000u) : bf16_bits_to_f32(m);
    else return m > 0xFFFFu ? __uint_as_float(0x7F800000u) : f16_bits_to_f32(m);
  }

  // Largest |x| of the tracked inputs (0 when none was added).
  __device__ __forceinline__ float max_abs() const {
    if constexpr (LDT == kLinF32) return __uint_as_float(hi());
    else if constexpr (LDT == kLinBF16) return bf16_bits_to_f32(hi());
    else return f16_bits_to_f32(hi());
  }

  // True when every tracked input is zero or has 2^-60 <= |x| < 2^60.
  __device__ __forceinline__ bool in_fast_range() const {
    if constexpr (LDT == kLinF32) {
      return lo() >= kFastLoBits - 1u && hi() < kFastHiBits;
    } else if constexpr (LDT == kLinBF16) {
      return lo() >= (kFastLoBits >> 16) - 1u && hi() < (kFastHiBits >> 16);
    } else {
      return hi() < 0x7C00u;  // every finite fp16 value is zero or within [2^-24, 65504]
    }
  }
};

}  // namespace kvhip
