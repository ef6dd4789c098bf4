// common.hpp -- shared device helpers and host-side error plumbing for libcsahca.
//
// Written for gfx950 (CDNA4): 64-lane wavefronts, 16-byte global loads, fp32
// math in VALU.  Softmax state is kept in the base-2 domain (scores pre-scaled
// by log2(e)) so every exponential is one v_exp_f32.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <type_traits>

#include "csahca.h"

namespace csahca {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Storage types
// ---------------------------------------------------------------------------
struct bf16 {
  uint16_t bits;
};
using f16 = _Float16;

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 with round-to-nearest-even (NaN stays NaN).
__device__ __forceinline__ uint16_t float_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u) {
    if (u & 0x007fffffu) u |= 0x00400000u;
    return static_cast<uint16_t>(u >> 16);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(double x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(f16 x) { return static_cast<float>(x); }
__device__ __forceinline__ float to_f32(bf16 x) { return bf16_bits_to_float(x.bits); }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <>
__device__ __forceinline__ double from_f32<double>(float x) { return static_cast<double>(x); }
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) { return static_cast<f16>(x); }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return bf16{float_to_bf16_bits(x)}; }

// Number of T elements in one 16-byte load.
template <typename T>
struct Vec16 {
  static constexpr int N = 16 / static_cast<int>(sizeof(T));
};

// Load 16 bytes (N elements of T) and widen to fp32.  p must be 16-byte aligned.
template <typename T>
__device__ __forceinline__ void load16(const T* __restrict__ p, float* out);

template <>
__device__ __forceinline__ void load16<bf16>(const bf16* __restrict__ p, float* out) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t v[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(v[i] << 16);
    out[2 * i + 1] = __uint_as_float(v[i] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void load16<f16>(const f16* __restrict__ p, float* out) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 w = *reinterpret_cast<const h8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) out[i] = static_cast<float>(w[i]);
}

template <>
__device__ __forceinline__ void load16<float>(const float* __restrict__ p, float* out) {
  const float4 w = *reinterpret_cast<const float4*>(p);
  out[0] = w.x;
  out[1] = w.y;
  out[2] = w.z;
  out[3] = w.w;
}

template <>
__device__ __forceinline__ void load16<double>(const double* __restrict__ p, float* out) {
  const double2 w = *reinterpret_cast<const double2*>(p);
  out[0] = static_cast<float>(w.x);
  out[1] = static_cast<float>(w.y);
}

// Widen 16 loaded bytes of T to fp32 (N = 16/sizeof(T) values).
template <typename T>
__device__ __forceinline__ void widen16(const uint4 w, float* out);
template <>
__device__ __forceinline__ void widen16<bf16>(const uint4 w, float* out) {
  const uint32_t x[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = __uint_as_float(x[i] << 16);
    out[2 * i + 1] = __uint_as_float(x[i] & 0xffff0000u);
  }
}
template <>
__device__ __forceinline__ void widen16<f16>(const uint4 w, float* out) {
  const uint32_t x[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x[i] & 0xffffu)));
    out[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(x[i] >> 16)));
  }
}
template <>
__device__ __forceinline__ void widen16<float>(const uint4 w, float* out) {
  out[0] = __uint_as_float(w.x);
  out[1] = __uint_as_float(w.y);
  out[2] = __uint_as_float(w.z);
  out[3] = __uint_as_float(w.w);
}
template <>
__device__ __forceinline__ void widen16<double>(const uint4 w, float* out) {
  out[0] = static_cast<float>(__builtin_bit_cast(double, (static_cast<uint64_t>(w.y) << 32) | w.x));
  out[1] = static_cast<float>(__builtin_bit_cast(double, (static_cast<uint64_t>(w.w) << 32) | w.z));
}

// One unconditional global load from an address the compiler cannot see
// through (an empty asm launders it): selects of addresses stay selects, and
// no load ends up under a per-lane branch, where the wait-count pass would
// make every load in flight complete at the join and so serialise a batch of
// loads meant to overlap.
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <typename V>
__device__ __forceinline__ V load_global_raw(const void* p) {
  uint64_t a = reinterpret_cast<uint64_t>(p);
  asm volatile("" : "+v"(a));
  return *reinterpret_cast<const __attribute__((address_space(1))) V*>(a);
}
__device__ __forceinline__ int32_t load_global_i32(const void* p) { return load_global_raw<int32_t>(p); }
__device__ __forceinline__ uint2 load_global_u2(const void* p) {
  const u32x2_t v = load_global_raw<u32x2_t>(p);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint4 load_global_u4(const void* p) {
  const u32x4_t v = load_global_raw<u32x4_t>(p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
// One element of a storage type (2, 4 or 8 bytes), through an integer load.
template <typename T>
__device__ __forceinline__ T load_global_elem(const T* p) {
  using U = std::conditional_t<sizeof(T) == 2, uint16_t, std::conditional_t<sizeof(T) == 4, uint32_t, uint64_t>>;
  static_assert(sizeof(T) == sizeof(U), "2, 4 or 8 byte storage types");
  const U u = load_global_raw<U>(p);
  T t;
  __builtin_memcpy(&t, &u, sizeof(T));
  return t;
}

// Four consecutive elements of T at p (aligned to 4 * sizeof(T)) widened to
// fp32, through unconditional loads of 8, 16 or 2 x 16 bytes.
template <typename T>
__device__ __forceinline__ void load4_f32(const T* p, float* out) {
  float tmp[8];
  if constexpr (sizeof(T) == 2) {
    const uint2 t = load_global_u2(p);
    widen16<T>(make_uint4(t.x, t.y, 0u, 0u), tmp);
  } else if constexpr (sizeof(T) == 4) {
    widen16<T>(load_global_u4(p), tmp);
  } else {
    const uint4 lo = load_global_u4(p), hi = load_global_u4(p + 2);
    widen16<T>(lo, tmp);
    widen16<T>(hi, tmp + 2);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = tmp[e];
}

// Store N = 16/sizeof(T) values; p 16-byte aligned.
template <typename T>
__device__ __forceinline__ void store16(T* __restrict__ p, const float* v) {
  constexpr int N = Vec16<T>::N;
#pragma unroll
  for (int i = 0; i < N; ++i) p[i] = from_f32<T>(v[i]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Butterfly sums / maxima over lane groups (masks are XOR distances).
// Value held by lane (lane ^ D), D a power of two below 64, with no LDS
// traffic: DPP quad permutes for 1 and 2, a half-row mirror (lane ^ 7) then a
// quad reverse (lane ^ 3) for 4, a row rotate by 8 for 8, and the gfx950 row
// swaps for 16 and 32 (v_permlane16/32_swap exchange the odd half of the first
// operand with the even half of the second, so with both operands = x the
// first result holds the even rows twice and the second the odd rows twice).
template <int Ctrl>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t x) {
  return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(x), Ctrl, 0xF, 0xF, false));
}

template <int D>
__device__ __forceinline__ uint32_t lane_xor(uint32_t x, int lane) {
  if constexpr (D == 1) {
    return dpp_mov<0xB1>(x);  // quad_perm [1,0,3,2]
  } else if constexpr (D == 2) {
    return dpp_mov<0x4E>(x);  // quad_perm [2,3,0,1]
  } else if constexpr (D == 4) {
    return dpp_mov<0x1B>(dpp_mov<0x141>(x));  // quad_perm [3,2,1,0] after row_half_mirror
  } else if constexpr (D == 8) {
    return dpp_mov<0x128>(x);  // row_ror:8
  } else if constexpr (D == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    static_assert(D == 32, "lane_xor: D must be a power of two below 64");
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}

// Wavefront-local ordering point for LDS traffic between lanes of one wavefront.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __builtin_amdgcn_wave_barrier();
}

// Workgroup barrier that orders LDS traffic only.  Global loads issued before
// it stay in flight (__syncthreads() also waits for every outstanding global
// access), so a kernel can prefetch across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Cross-workgroup words without cache maintenance: a 32-bit value travels in
// a 64-bit word (tag << 32 | value), written and read with device-scope atomic
// stores / loads, which are coherent across XCDs on their own.  A reader
// accepts a word once it carries the tag it expects, so no fence orders it.
__device__ __forceinline__ void put_tagged(uint64_t* p, uint32_t tag, uint32_t v) {
  __hip_atomic_store(p, (static_cast<uint64_t>(tag) << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint64_t get_raw(const uint64_t* p) {
  return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Launch epochs of a tagged exchange: an epoch word per exchange group holds
// the tag of the last completed launch; kPoisonEpoch marks a group whose
// exchange timed out (every later launch on it skips its waits and writes NaN
// until the words are zero-filled again).
constexpr uint32_t kPoisonEpoch = 0xffffffffu;

// This launch's tag for a group whose epoch word reads `epoch` (never the
// poison value; after 2^32 - 2 launches the sequence restarts at 1, and every
// exchanged word is rewritten by each launch, so no stale word carries it).
__device__ __forceinline__ uint32_t launch_tag(uint32_t epoch) {
  const uint32_t t = epoch + 1u;
  return t == kPoisonEpoch ? 1u : t;
}

// Value of lane (lane ^ off), off in {1, 2, 4, 8, 16, 32} (a constant once the
// caller's loop is unrolled): DPP / row-swap moves, no LDS round trip.  The
// whole wavefront must be active.
__device__ __forceinline__ float xor_lanes(float v, int off) {
  const int lane = static_cast<int>(__lane_id());
  const uint32_t u = __float_as_uint(v);
  switch (off) {
    case 1: return __uint_as_float(lane_xor<1>(u, lane));
    case 2: return __uint_as_float(lane_xor<2>(u, lane));
    case 4: return __uint_as_float(lane_xor<4>(u, lane));
    case 8: return __uint_as_float(lane_xor<8>(u, lane));
    case 16: return __uint_as_float(lane_xor<16>(u, lane));
    default: return __uint_as_float(lane_xor<32>(u, lane));
  }
}

// Sums each of the N values v[0..N) over the L lanes of the lane's aligned
// group of L (N <= L, both powers of two), transposed: every exchange carries
// values another lane needs, so log2(N) halving steps leave each lane with one
// value, then plain steps finish it.  Lane l ends with the sum of value
// (l % L) / (L / N).  Every sum is formed by the same pairwise tree (own +
// partner at distances L/2, L/4, ..., 1) as a butterfly over each value, so
// the bits are those of the butterfly; it takes N - 1 + log2(L / N)
// exchanges instead of N log2(L).
template <int N, int L>
__device__ __forceinline__ float transposed_group_sum(float (&v)[N]) {
  static_assert(N >= 1 && N <= L && L <= kWave && (N & (N - 1)) == 0 && (L & (L - 1)) == 0,
                "transposed_group_sum: N <= L, powers of two");
  const int lane = static_cast<int>(__lane_id());
#pragma unroll
  for (int half = N / 2, d = L / 2; half >= 1; half /= 2, d /= 2) {
    // Bit-mask selects (v_bfi): a ternary over two array elements is turned by
    // the compiler into a dynamically indexed read of the whole array.
    const uint32_t up = (lane & d) ? 0xffffffffu : 0u;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const uint32_t lo = __float_as_uint(v[i]), hi = __float_as_uint(v[i + half]);
      const float send = __uint_as_float((lo & up) | (hi & ~up));
      const float keep = __uint_as_float((hi & up) | (lo & ~up));
      v[i] = keep + xor_lanes(send, d);
    }
  }
  float s = v[0];
#pragma unroll
  for (int d = L / (2 * N); d >= 1; d /= 2) s += xor_lanes(s, d);
  return s;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += xor_lanes(v, off);
  return v;
}

// ---------------------------------------------------------------------------
// Host helpers
// ---------------------------------------------------------------------------
int fail(int code, const char* msg);
int fail_hip(hipError_t err, const char* where);
// Compute units of the current device (cached per device; 0 if the query fails).
int device_cu_count();
void clear_error();

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

inline bool valid_dtype(int dt) {
  return dt == CSAHCA_F32 || dt == CSAHCA_F16 || dt == CSAHCA_BF16 || dt == CSAHCA_F64;
}

// Dispatch a callable templated on the storage type.
template <typename F>
int dispatch_dtype(int dtype, F&& f) {
  switch (dtype) {
    case CSAHCA_BF16: return f(bf16{});
    case CSAHCA_F16: return f(f16{});
    case CSAHCA_F32: return f(float{});
    case CSAHCA_F64: return f(double{});
    default: return fail(CSAHCA_ERR_ARGUMENT, "unsupported dtype");
  }
}

#define CSAHCA_REQUIRE(cond, msg)                                   \
  do {                                                              \
    if (!(cond)) return ::csahca::fail(CSAHCA_ERR_ARGUMENT, (msg)); \
  } while (0)

// Launch-time profiling (csahca_profile_begin/end): while active on the
// calling thread, launches go through hipExtLaunchKernelGGL with a start/stop
// event pair, which timestamps the dispatch itself.
bool profiling_active();
bool profile_take_events(hipEvent_t* start, hipEvent_t* stop);
void profile_record(const char* name, hipEvent_t start, hipEvent_t stop);

template <typename... KArgs, typename... Args>
int launch(const char* name, void (*kernel)(KArgs...), dim3 grid, dim3 block, size_t shmem,
           hipStream_t stream, Args... args) {
  if (profiling_active()) {
    hipEvent_t a = nullptr, b = nullptr;
    if (!profile_take_events(&a, &b)) return fail(CSAHCA_ERR_HIP, "profiling: hipEventCreate failed");
    hipExtLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(shmem), stream, a, b, 0u,
                          static_cast<KArgs>(args)...);
    profile_record(name, a, b);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, static_cast<uint32_t>(shmem), stream,
                       static_cast<KArgs>(args)...);
  }
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail_hip(e, name);
  return CSAHCA_OK;
}

#define CSAHCA_LAUNCH_CHECK(where)                                 \
  do {                                                             \
    hipError_t e_ = hipGetLastError();                             \
    if (e_ != hipSuccess) return ::csahca::fail_hip(e_, (where));  \
  } while (0)

}  // namespace csahca
