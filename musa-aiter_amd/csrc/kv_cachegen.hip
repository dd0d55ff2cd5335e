// CacheGen-style uniform-bin KV codec for MI355X (gfx950).
//
// Encode turns a floating tensor into one uint8 bin per element over the
// tensor's own [min, max] range, plus a dequant codebook and the empirical
// CDF of the bins.  It is three launches and no host synchronisation:
//
//   1. cg_minmax_kernel -- one pass over the input; each workgroup writes its
//                          (min, max) pair to the workspace; workgroup 0 also
//                          clears the bin counters.
//   2. cg_encode_kernel -- every workgroup folds the pairs into the range (a
//                          few KiB from L2) and derives the scale; workgroup 0
//                          writes the codebook (torch.linspace's arithmetic);
//                          all write the bins and count them in per-wave LDS
//                          histograms, added to 64-bit global counters once
//                          per workgroup.
//   3. cg_cdf_kernel    -- one workgroup: the counters into the CDF.
//
// The input is read twice (the range must be known before any bin is), the
// bins written once: 2 * elem + 1 bytes per element.  Decode is one launch:
// a gather through a <= 256-entry table staged in LDS, 1 + E bytes per element.
// The streaming kernels walk contiguous chunks (layout below): the range and
// bin passes on 1024 persistent workgroups, which keeps the per-workgroup
// range fold and the global counter updates small (the bin pass prefetches
// its next chunk), decode on one chunk per workgroup.
//
// Arithmetic follows the reference's torch path step by step, each float32
// operation rounded on its own (the library is built without contraction):
// scale = (1 / (max - min)) * (num_bins - 1), bin = rint((x - min) * scale),
// clamped.  The reference's native kernel rounds differently, with a
// double-precision scale and trunc((x - min) * scale + 0.5) as one fused
// multiply-add; `native` selects it.
#include <math.h>

#include "kv_hip_common.h"
#include "kv_launch.h"

namespace kvhip {

namespace {

// The streaming kernels visit the 16-byte vectors of their wide side in chunks of
// kWavesPerBlock * kWave * V vectors: inside a chunk, lane l of wave w takes vectors
// base + w * kWave * V + k * kWave + l (k < V), so each of a wave's V loads or stores covers
// 1 KiB contiguously and the wave's V KiB are contiguous too; workgroup g takes chunks g,
// g + grid, ...  Measured on MI355X over 1 GiB, this shape reads at 7.0 TB/s where a grid-stride
// loop with four loads per thread spread a grid apart reads at 5.3 TB/s.  Grid caps and V per
// kernel come from a sweep over 1024-8192 workgroups and 2-8 vectors.
#ifndef KVHIP_CG_MINMAX_GROUPS
#define KVHIP_CG_MINMAX_GROUPS 1024
#endif
#ifndef KVHIP_CG_ENCODE_GROUPS
#define KVHIP_CG_ENCODE_GROUPS 1024
#endif
#ifndef KVHIP_CG_DECODE_GROUPS
#define KVHIP_CG_DECODE_GROUPS (1 << 22)
#endif
constexpr int kCgMinmaxGroups = KVHIP_CG_MINMAX_GROUPS;
constexpr int kCgEncodeGroups = KVHIP_CG_ENCODE_GROUPS;
constexpr int kCgDecodeGroups = KVHIP_CG_DECODE_GROUPS;
#ifndef KVHIP_CG_ENCODE_VECS
#define KVHIP_CG_ENCODE_VECS 4
#endif
constexpr int kCgMinmaxVecs = 4;
constexpr int kCgEncodeVecs = KVHIP_CG_ENCODE_VECS;
constexpr int kCgDecodeVecs = 4;
// Histogram copies per wave: lane l counts into copy l % kCgHistCopies, so lanes of one
// instruction that hit the same bin use different LDS banks.
constexpr int kCgHistCopies = 4;

// Calls f(k, vector) for the vectors of chunk c below `slots`; a full chunk (all but the last)
// takes no per-lane bounds test.
template <int V, class F>
__device__ __forceinline__ void for_chunk(int64_t c, int64_t per_chunk, int64_t lane_off, int64_t slots, F&& f) {
  const int64_t base = c * per_chunk + lane_off;
  if ((c + 1) * per_chunk <= slots) {
#pragma unroll
    for (int k = 0; k < V; ++k) f(k, base + k * kWave);
  } else {
#pragma unroll
    for (int k = 0; k < V; ++k)
      if (base + k * kWave < slots) f(k, base + k * kWave);
  }
}

// Workspace layout: the 256 bin counters, the per-workgroup (min, max) pairs.
constexpr int64_t kCgCountsOffset = 0;
constexpr int64_t kCgPairsOffset = 4096;
static_assert(kCgCountsOffset + 256 * 8 <= kCgPairsOffset, "workspace layout");
static_assert(kCgPairsOffset + int64_t{kCgMinmaxGroups} * 8 <= kCacheGenWorkspaceBytes, "workspace too small");

template <int IN>
struct CgIn;
template <>
struct CgIn<kCgF32> { static constexpr int kBytes = 4; };
template <>
struct CgIn<kCgF16> { static constexpr int kBytes = 2; };
template <>
struct CgIn<kCgBF16> { static constexpr int kBytes = 2; };
template <>
struct CgIn<kCgF64> { static constexpr int kBytes = 8; };

// Element j of a 16-byte slot, widened (or for float64 rounded) to float32 as tensor.float() does.
template <int IN>
__device__ __forceinline__ float cg_elem(const u32x4& v, int j) {
  if constexpr (IN == kCgF32) {
    return __uint_as_float(v[j]);
  } else if constexpr (IN == kCgF16) {
    return f16_bits_to_f32(half_of(v[j >> 1], j & 1));
  } else if constexpr (IN == kCgBF16) {
    return bf16_bits_to_f32(half_of(v[j >> 1], j & 1));
  } else {
    const uint64_t bits = static_cast<uint64_t>(v[2 * j]) | (static_cast<uint64_t>(v[2 * j + 1]) << 32);
    return static_cast<float>(__longlong_as_double(static_cast<long long>(bits)));
  }
}

template <int IN>
__device__ __forceinline__ float cg_load1(const uint8_t* x, int64_t i) {
  if constexpr (IN == kCgF32) {
    return reinterpret_cast<const float*>(x)[i];
  } else if constexpr (IN == kCgF16) {
    return f16_bits_to_f32(reinterpret_cast<const uint16_t*>(x)[i]);
  } else if constexpr (IN == kCgBF16) {
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(x)[i]);
  } else {
    return static_cast<float>(reinterpret_cast<const double*>(x)[i]);
  }
}

// Running (min, max) with NaN propagation (torch's min / max return NaN if any element is).
struct MinMax {
  float mn = INFINITY;
  float mx = -INFINITY;
  bool nan = false;
  __device__ __forceinline__ void fold(float f) {
    nan |= f != f;
    mn = fminf(mn, f);
    mx = fmaxf(mx, f);
  }
};

// Folds a MinMax over the workgroup; every thread returns the result.
__device__ __forceinline__ MinMax block_minmax(MinMax m) {
  __shared__ float s_mn[kWavesPerBlock], s_mx[kWavesPerBlock];
  __shared__ int s_nan[kWavesPerBlock];
  for (int off = kWave / 2; off > 0; off >>= 1) {
    m.mn = fminf(m.mn, __shfl_xor(m.mn, off));
    m.mx = fmaxf(m.mx, __shfl_xor(m.mx, off));
  }
  const bool any_nan = ballot(m.nan) != 0;
  const int w = wave_in_block();
  if (lane_id() == 0) {
    s_mn[w] = m.mn;
    s_mx[w] = m.mx;
    s_nan[w] = any_nan ? 1 : 0;
  }
  __syncthreads();
  MinMax r;
  for (int i = 0; i < kWavesPerBlock; ++i) {
    r.mn = fminf(r.mn, s_mn[i]);
    r.mx = fmaxf(r.mx, s_mx[i]);
    r.nan |= s_nan[i] != 0;
  }
  __syncthreads();
  if (r.nan) r.mn = r.mx = __builtin_nanf("");
  return r;
}

template <int IN, bool VEC>
__global__ __launch_bounds__(kBlockThreads) void cg_minmax_kernel(const uint8_t* __restrict__ x, int64_t n,
                                                                  float2* __restrict__ pairs,
                                                                  uint64_t* __restrict__ counts) {
  constexpr int kEps = 16 / CgIn<IN>::kBytes;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kBlockThreads + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlockThreads;
  MinMax m;
  int64_t first_scalar = 0;
  if constexpr (VEC) {
    constexpr int V = kCgMinmaxVecs;
    const int64_t slots = n / kEps;
    const int64_t per_chunk = int64_t{kBlockThreads} * V;
    const int64_t lane_off = int64_t{wave_in_block()} * kWave * V + lane_id();
    for (int64_t c = blockIdx.x; c * per_chunk < slots; c += gridDim.x) {
      u32x4 v[V];
      for_chunk<V>(c, per_chunk, lane_off, slots, [&](int k, int64_t s) { v[k] = ld16(x + s * 16); });
      for_chunk<V>(c, per_chunk, lane_off, slots, [&](int k, int64_t) {
#pragma unroll
        for (int j = 0; j < kEps; ++j) m.fold(cg_elem<IN>(v[k], j));
      });
    }
    first_scalar = slots * kEps;
  }
  for (int64_t i = first_scalar + tid; i < n; i += stride) m.fold(cg_load1<IN>(x, i));
  const MinMax r = block_minmax(m);
  if (threadIdx.x == 0) pairs[blockIdx.x] = make_float2(r.mn, r.mx);
  if (blockIdx.x == 0) counts[threadIdx.x] = 0;  // kBlockThreads == 256 counters
}

struct CgEncodeArgs {
  const uint8_t* x;
  uint8_t* enc;
  int64_t n;
  const float2* pairs;  // null: min_arg / scale_arg given by the caller, no histogram
  int32_t num_pairs;
  uint64_t* counts;
  float* codebook;
  int32_t num_bins;
  float min_arg;
  float scale_arg;
};

// codebook[t]: torch.full(min) for a constant range, else torch.linspace(min, max, nb) -- step in
// float32, the first half counted up from start and the second half down from end, one fused
// multiply-add each.
__device__ __forceinline__ float cg_codebook(float mn, float mx, int nb, int t) {
  if (mx == mn) return mn;
  const float step = (mx - mn) / static_cast<float>(nb - 1);
  return t < nb / 2 ? __builtin_fmaf(step, static_cast<float>(t), mn)
                    : __builtin_fmaf(-step, static_cast<float>(nb - 1 - t), mx);
}

// Clamping is fminf(fmaxf(v, 0), top): fmaxf returns the non-NaN operand, so NaN gives bin 0, and
// the float -> uint conversion truncates (exact for the rounded torch-path value).
template <bool NATIVE>
__device__ __forceinline__ uint32_t cg_bin(float x, float mn, float scale, float top) {
  const float t = x - mn;
  if constexpr (NATIVE) {
    const float v = __builtin_fmaf(t, scale, 0.5f);
    return static_cast<uint32_t>(fminf(fmaxf(v, 0.0f), top));
  } else {
    return static_cast<uint32_t>(fminf(fmaxf(__builtin_rintf(t * scale), 0.0f), top));
  }
}

// cdf[0] = 0, cdf[t + 1] = (prefix of float32(count)) / numel, for the workgroup's 256 threads
// holding counts[t]: each count rounded to float32, prefix sums in double (exact: integers below
// 2**53), rounded to float32, divided by numel in float32.
__device__ __forceinline__ void cg_write_cdf(uint64_t count, int nb, int64_t numel, float* cdf) {
  __shared__ double scan[2][256];
  const int t = threadIdx.x;
  scan[0][t] = t < nb ? static_cast<double>(static_cast<float>(count)) : 0.0;
  __syncthreads();
  int cur = 0;
  for (int off = 1; off < 256; off <<= 1) {
    const double v = scan[cur][t] + (t >= off ? scan[cur][t - off] : 0.0);
    scan[cur ^ 1][t] = v;
    cur ^= 1;
    __syncthreads();
  }
  if (t == 0) cdf[0] = 0.0f;
  if (t < nb) cdf[t + 1] = static_cast<float>(scan[cur][t]) / static_cast<float>(numel);
}

template <int IN, bool NATIVE, bool HIST, bool VEC>
__global__ __launch_bounds__(kBlockThreads) void cg_encode_kernel(CgEncodeArgs a) {
  constexpr int kEps = 16 / CgIn<IN>::kBytes;
  __shared__ uint32_t hist[kWavesPerBlock][256 * kCgHistCopies];
  const int nb = a.num_bins;
  float mn = a.min_arg, scale = a.scale_arg;
  if constexpr (HIST) {
    MinMax m;
    for (int i = threadIdx.x; i < a.num_pairs; i += kBlockThreads) {
      const float2 p = a.pairs[i];
      m.fold(p.x);
      m.fold(p.y);
    }
    const MinMax r = block_minmax(m);
    mn = r.mn;
    if constexpr (NATIVE) {
      scale = static_cast<float>(static_cast<double>(nb - 1) /
                                 (static_cast<double>(r.mx) - static_cast<double>(r.mn)));
    } else {
      const float recip = 1.0f / (r.mx - r.mn);
      scale = recip * static_cast<float>(nb - 1);
    }
    if (r.mx == r.mn) scale = 0.0f;  // constant tensor: every bin is 0
    if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < nb)
      a.codebook[threadIdx.x] = cg_codebook(r.mn, r.mx, nb, threadIdx.x);
    for (int i = threadIdx.x; i < kWavesPerBlock * 256 * kCgHistCopies; i += kBlockThreads) (&hist[0][0])[i] = 0;
    __syncthreads();
  }
  const float top = static_cast<float>(nb - 1);
  uint32_t* my_hist = hist[wave_in_block()] + (lane_id() & (kCgHistCopies - 1));
  auto count = [&](uint32_t b, uint32_t inc) {
    if constexpr (HIST) atomicAdd(&my_hist[b * kCgHistCopies], inc);
  };
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kBlockThreads + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlockThreads;
  int64_t first_scalar = 0;
  if constexpr (VEC) {
    const int64_t slots = a.n / kEps;
    auto emit = [&](int64_t s, const u32x4& v) {
      uint32_t b[kEps];
      bool same = true;
#pragma unroll
      for (int j = 0; j < kEps; ++j) {
        b[j] = cg_bin<NATIVE>(cg_elem<IN>(v, j), mn, scale, top);
        same &= b[j] == b[0];
      }
      // A run of equal bins (constant regions, zero padding) is one LDS update, not kEps.
      if (same) {
        count(b[0], kEps);
      } else {
#pragma unroll
        for (int j = 0; j < kEps; ++j) count(b[j], 1u);
      }
      uint8_t* d = a.enc + s * kEps;
      if constexpr (kEps == 8) {
        u32x2 w;
        w[0] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
        w[1] = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
        stv<8>(d, w);
      } else if constexpr (kEps == 4) {
        stv<4>(d, b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24));
      } else {
        stv<2>(d, static_cast<uint16_t>(b[0] | (b[1] << 8)));
      }
    };
    // Software-pipelined: the next chunk's vectors are loaded before this chunk's bins are
    // computed and stored, so each wave keeps 2 * V vectors in flight.
    constexpr int V = kCgEncodeVecs;
    const int64_t per_chunk = int64_t{kBlockThreads} * V;
    const int64_t lane_off = int64_t{wave_in_block()} * kWave * V + lane_id();
    auto load = [&](int64_t c, u32x4* v) {
      for_chunk<V>(c, per_chunk, lane_off, slots, [&](int k, int64_t s) { v[k] = ld16(a.x + s * 16); });
    };
    u32x4 cur[V], nxt[V];
    int64_t c = blockIdx.x;
    if (c * per_chunk < slots) load(c, cur);
    for (; c * per_chunk < slots; c += gridDim.x) {
      const int64_t cn = c + gridDim.x;
      if (cn * per_chunk < slots) load(cn, nxt);
      for_chunk<V>(c, per_chunk, lane_off, slots, [&](int k, int64_t s) { emit(s, cur[k]); });
#pragma unroll
      for (int k = 0; k < V; ++k) cur[k] = nxt[k];
    }
    first_scalar = slots * kEps;
  }
  for (int64_t i = first_scalar + tid; i < a.n; i += stride) {
    const uint32_t b = cg_bin<NATIVE>(cg_load1<IN>(a.x, i), mn, scale, top);
    count(b, 1u);
    a.enc[i] = static_cast<uint8_t>(b);
  }
  if constexpr (HIST) {
    __syncthreads();
    const int t = threadIdx.x;
    if (t < nb) {
      uint32_t sum = 0;
#pragma unroll
      for (int w = 0; w < kWavesPerBlock; ++w)
#pragma unroll
        for (int c = 0; c < kCgHistCopies; ++c) sum += hist[w][t * kCgHistCopies + c];
      if (sum != 0)
        atomicAdd(reinterpret_cast<unsigned long long*>(&a.counts[t]), static_cast<unsigned long long>(sum));
    }
  }
}

// One workgroup, after cg_encode_kernel: the counters into cdf[num_bins + 1].  (Finishing in the
// encode kernel's last workgroup would need a device-scope release fence in every workgroup,
// which writes back L2 and costs far more than this launch.)
__global__ __launch_bounds__(kBlockThreads) void cg_cdf_kernel(const uint64_t* __restrict__ counts, int32_t nb,
                                                               int64_t numel, float* __restrict__ cdf) {
  const int t = threadIdx.x;
  cg_write_cdf(t < nb ? counts[t] : 0, nb, numel, cdf);
}

struct CgDecodeArgs {
  const uint8_t* codes;
  uint8_t* out;
  int64_t n;
  const uint8_t* table;  // table_len entries of E bytes, aligned to E
  int32_t table_len;
  int32_t* max_code;     // CHECK: largest code seen (atomic max)
};

template <int E>
struct Entry;
template <>
struct Entry<1> { using T = uint8_t; };
template <>
struct Entry<2> { using T = uint16_t; };
template <>
struct Entry<4> { using T = uint32_t; };
template <>
struct Entry<8> { using T = uint64_t; };
template <>
struct Entry<16> { using T = u32x4; };

// Decode through a table staged in LDS (GLOBAL_TABLE: read from global memory, the reference
// kernel's access, for callers that do not pass the table length).
template <int E, bool VEC, bool CHECK, bool GLOBAL_TABLE>
__global__ __launch_bounds__(kBlockThreads) void cg_decode_kernel(CgDecodeArgs a) {
  using T = typename Entry<E>::T;
  constexpr int kCodes = 16 / E;  // codes per 16-byte output slot
  __shared__ T tab[GLOBAL_TABLE ? 1 : 256];
  const T* table;
  if constexpr (GLOBAL_TABLE) {
    table = reinterpret_cast<const T*>(a.table);
  } else {
    const T* g = reinterpret_cast<const T*>(a.table);
    for (int i = threadIdx.x; i < 256; i += kBlockThreads) tab[i] = i < a.table_len ? g[i] : T{};
    __syncthreads();
    table = tab;
  }
  uint32_t top = 0;
  auto look = [&](uint32_t c) -> T {
    if constexpr (CHECK) top = top > c ? top : c;
    return table[c];
  };
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kBlockThreads + threadIdx.x;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlockThreads;
  int64_t first_scalar = 0;
  if constexpr (VEC) {
    const int64_t slots = a.n / kCodes;
    using C = typename VecType<kCodes>::T;
    auto emit = [&](int64_t s, C cw) {
      u32x4 o;
      if constexpr (E == 16) {
        o = look(static_cast<uint32_t>(cw));
      } else if constexpr (E == 8) {
        const uint32_t w = cw;
        const uint64_t lo = look(w & 0xFFu), hi = look((w >> 8) & 0xFFu);
        o[0] = static_cast<uint32_t>(lo);
        o[1] = static_cast<uint32_t>(lo >> 32);
        o[2] = static_cast<uint32_t>(hi);
        o[3] = static_cast<uint32_t>(hi >> 32);
      } else if constexpr (E == 4) {
        const uint32_t w = cw;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = look((w >> (8 * j)) & 0xFFu);
      } else if constexpr (E == 2) {
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            const uint32_t w = cw[k];
            o[2 * k + j] = static_cast<uint32_t>(look((w >> (16 * j)) & 0xFFu)) |
                           (static_cast<uint32_t>(look((w >> (16 * j + 8)) & 0xFFu)) << 16);
          }
      } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const uint32_t w = cw[k];
          o[k] = static_cast<uint32_t>(look(w & 0xFFu)) | (static_cast<uint32_t>(look((w >> 8) & 0xFFu)) << 8) |
                 (static_cast<uint32_t>(look((w >> 16) & 0xFFu)) << 16) |
                 (static_cast<uint32_t>(look(w >> 24)) << 24);
        }
      }
      stv<16>(a.out + s * 16, o);
    };
    constexpr int V = kCgDecodeVecs;
    const int64_t per_chunk = int64_t{kBlockThreads} * V;
    const int64_t lane_off = int64_t{wave_in_block()} * kWave * V + lane_id();
    // (A per-lane bounds test on every vector measures faster here than separate full-chunk code.)
    for (int64_t ch = blockIdx.x; ch * per_chunk < slots; ch += gridDim.x) {
      const int64_t base = ch * per_chunk + lane_off;
      const bool full = (ch + 1) * per_chunk <= slots;
      C cw[V];
#pragma unroll
      for (int k = 0; k < V; ++k)
        if (full || base + k * kWave < slots) cw[k] = ldv<kCodes>(a.codes + (base + k * kWave) * kCodes);
#pragma unroll
      for (int k = 0; k < V; ++k)
        if (full || base + k * kWave < slots) emit(base + k * kWave, cw[k]);
    }
    first_scalar = slots * kCodes;
  }
  for (int64_t i = first_scalar + tid; i < a.n; i += stride)
    reinterpret_cast<T*>(a.out)[i] = look(a.codes[i]);
  if constexpr (CHECK) {
    for (int off = kWave / 2; off > 0; off >>= 1) {
      const uint32_t o = __shfl_xor(top, off);
      top = top > o ? top : o;
    }
    if (lane_id() == 0 && static_cast<int32_t>(top) >= a.table_len) atomicMax(a.max_code, static_cast<int>(top));
  }
}

// Workgroups for `units` vectors (or scalar elements) at `vecs` per thread, at most `cap`.
int cg_groups(int64_t units, int vecs, int cap) {
  const int64_t per_group = static_cast<int64_t>(kBlockThreads) * vecs;
  int64_t g = (units + per_group - 1) / per_group;
  if (g < 1) g = 1;
  if (g > cap) g = cap;
  return static_cast<int>(g);
}

template <int IN>
hipError_t encode_typed(const uint8_t* x, int64_t n, int nb, bool native, uint8_t* enc, float* codebook, float* cdf,
                        uint8_t* ws, hipStream_t stream) {
  constexpr int kEps = 16 / CgIn<IN>::kBytes;
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(enc) % kEps) == 0;
  const int64_t units = vec ? n / kEps : n;
  const int mgroups = cg_groups(units, kCgMinmaxVecs, kCgMinmaxGroups);
  const int groups = cg_groups(units, kCgEncodeVecs, kCgEncodeGroups);
  uint64_t* counts = reinterpret_cast<uint64_t*>(ws + kCgCountsOffset);
  float2* pairs = reinterpret_cast<float2*>(ws + kCgPairsOffset);
  if (vec)
    hipLaunchKernelGGL((cg_minmax_kernel<IN, true>), dim3(mgroups), dim3(kBlockThreads), 0, stream, x, n, pairs, counts);
  else
    hipLaunchKernelGGL((cg_minmax_kernel<IN, false>), dim3(mgroups), dim3(kBlockThreads), 0, stream, x, n, pairs,
                       counts);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  CgEncodeArgs a{x, enc, n, pairs, mgroups, counts, codebook, nb, 0.0f, 0.0f};
  if (native) {
    if (vec) hipLaunchKernelGGL((cg_encode_kernel<IN, true, true, true>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
    else hipLaunchKernelGGL((cg_encode_kernel<IN, true, true, false>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
  } else {
    if (vec) hipLaunchKernelGGL((cg_encode_kernel<IN, false, true, true>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
    else hipLaunchKernelGGL((cg_encode_kernel<IN, false, true, false>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
  }
  err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(cg_cdf_kernel, dim3(1), dim3(kBlockThreads), 0, stream, counts, nb, n, cdf);
  return hipGetLastError();
}

template <int E>
hipError_t decode_typed(const uint8_t* codes, int64_t n, const uint8_t* table, int table_len, uint8_t* out,
                        int32_t* max_code, hipStream_t stream) {
  constexpr int kCodes = 16 / E;
  const bool vec = (reinterpret_cast<uintptr_t>(codes) % kCodes) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
  const bool check = table_len < 256;
  const int groups = cg_groups(vec ? n / kCodes : n, kCgDecodeVecs, kCgDecodeGroups);
  CgDecodeArgs a{codes, out, n, table, table_len, max_code};
  if (vec) {
    if (check) hipLaunchKernelGGL((cg_decode_kernel<E, true, true, false>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
    else hipLaunchKernelGGL((cg_decode_kernel<E, true, false, false>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
  } else {
    if (check) hipLaunchKernelGGL((cg_decode_kernel<E, false, true, false>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
    else hipLaunchKernelGGL((cg_decode_kernel<E, false, false, false>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_cachegen_encode(const void* x, int in_dtype, int64_t n, int num_bins, bool native, uint8_t* enc,
                                  float* codebook, float* cdf, void* workspace, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const uint8_t* xs = static_cast<const uint8_t*>(x);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  switch (in_dtype) {
    case kCgF32: return encode_typed<kCgF32>(xs, n, num_bins, native, enc, codebook, cdf, ws, stream);
    case kCgF16: return encode_typed<kCgF16>(xs, n, num_bins, false, enc, codebook, cdf, ws, stream);
    case kCgBF16: return encode_typed<kCgBF16>(xs, n, num_bins, false, enc, codebook, cdf, ws, stream);
    case kCgF64: return encode_typed<kCgF64>(xs, n, num_bins, false, enc, codebook, cdf, ws, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_cachegen_bins(const float* x, uint8_t* enc, float min_val, float scale, int64_t n, int num_bins,
                                hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const uint8_t* xs = reinterpret_cast<const uint8_t*>(x);
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && (reinterpret_cast<uintptr_t>(enc) & 3) == 0;
  CgEncodeArgs a{xs, enc, n, nullptr, 0, nullptr, nullptr, num_bins, min_val, scale};
  const int groups = cg_groups(vec ? n / 4 : n, kCgEncodeVecs, kCgEncodeGroups);
  if (vec) hipLaunchKernelGGL((cg_encode_kernel<kCgF32, true, false, true>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
  else hipLaunchKernelGGL((cg_encode_kernel<kCgF32, true, false, false>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_cachegen_decode(const uint8_t* codes, int64_t n, const void* table, int table_len, int elem_bytes,
                                  void* out, int32_t* max_code, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const uint8_t* tb = static_cast<const uint8_t*>(table);
  uint8_t* o = static_cast<uint8_t*>(out);
  if (table_len < 0) {  // reference entry: float32 table of unknown length, read from global memory
    if (elem_bytes != 4) return hipErrorInvalidValue;
    const bool vec = (reinterpret_cast<uintptr_t>(codes) & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0;
    CgDecodeArgs a{codes, o, n, tb, 256, nullptr};
    const int groups = cg_groups(vec ? n / 4 : n, kCgDecodeVecs, kCgDecodeGroups);
    if (vec) hipLaunchKernelGGL((cg_decode_kernel<4, true, false, true>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
    else hipLaunchKernelGGL((cg_decode_kernel<4, false, false, true>), dim3(groups), dim3(kBlockThreads), 0, stream, a);
    return hipGetLastError();
  }
  if (table_len < 1 || table_len > 256 || (table_len < 256 && max_code == nullptr)) return hipErrorInvalidValue;
  switch (elem_bytes) {
    case 1: return decode_typed<1>(codes, n, tb, table_len, o, max_code, stream);
    case 2: return decode_typed<2>(codes, n, tb, table_len, o, max_code, stream);
    case 4: return decode_typed<4>(codes, n, tb, table_len, o, max_code, stream);
    case 8: return decode_typed<8>(codes, n, tb, table_len, o, max_code, stream);
    case 16: return decode_typed<16>(codes, n, tb, table_len, o, max_code, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kvhip
