// dsv4_pack.hip -- quantize-on-write of BF16 latent tokens into the DSV4 paged
// FP8 cache, for gfx950.
//
// Format and rule (hybrid_attention/dsv4_correctness.py:19-59): token loc
// lives on page loc / page_size at row loc % page_size of 576 bytes -- 448 OCP
// e4m3fn "nope" bytes, then the 64 bf16 "rope" values verbatim -- and its 7
// scale bytes sit after the page's rows, 8 bytes per token.  Per 64-value
// tile: max_abs = max(|v|, 1e-8) (fp32), r = max_abs / 448 (fp32), exponent
// E = ceil(log2 r), scale byte = clamp(E + 127, 0, 255), stored value =
// e4m3fn_rne(clamp(v / 2^E, -448, 448)).  Exactly the bytes the reference
// writes are written (not the scale pad byte, not the page padding).
//
// A wavefront packs a token at a time: lanes 0..55 own 8 nope values each
// (tile = lane / 8, so a tile's max is a reduction over 8 adjacent lanes),
// lanes 56..63 copy 16 bytes of rope each.
#include "common.hpp"

#include <climits>

namespace csahca {
namespace {

constexpr int kPackNope = 448;
constexpr int kPackRowBytes = kPackNope + 2 * 64;  // 576
constexpr int kPackScaleBytes = 8;
constexpr int kPackWaves = 4;          // wavefronts per workgroup
constexpr int kPackTokensPerWave = 1;  // tokens per wavefront (4 measured slower: 30.6 vs 28.2 us / 65536)

// Four clamped fp32 values -> four OCP e4m3fn bytes (byte i = value i), round
// to nearest even, on the gfx950 conversion v_cvt_pk_fp8_f32.  The values this
// kernel converts are v / 2^E clamped to [-448, 448], v bf16 and 2^E exact:
// bf16 values in that range, or values that round to +-0.  On all of them the
// instruction gives the bytes of the integer rounding it replaces (keep 3
// mantissa bits of the fp32 encoding with RNE on the dropped 20 bits; a
// quantum of 2^-9 below 2^-6): checked on the device over every bf16 bit
// pattern and tiny fp32 values, and pinned here by the oracle comparisons of
// every finite bf16 value in range (tests/test_gpu_dsv4_pack.py).
__device__ __forceinline__ uint32_t e4m3fn_rne4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true));
}

// ceil(log2(r)) for a positive finite fp32 r, exactly.
__device__ __forceinline__ int ceil_log2(float r) {
  int e;
  const float m = frexpf(r, &e);  // r = m 2^e, m in [0.5, 1)
  return m == 0.5f ? e - 1 : e;
}

// Quantise and store one token whose 16 bytes of this lane are `w` (see the
// lane layout above).
template <bool kVec>
__device__ __forceinline__ void pack_token(const uint4 w, int64_t loc, int lane, uint8_t* __restrict__ cache,
                                           int64_t num_pages, int64_t bpp, int page_size) {
  if (loc < 0) return;
  // 32-bit division whenever the slot fits (always, for an int32 slot list).
  const int64_t page = loc <= static_cast<int64_t>(UINT32_MAX)
                           ? static_cast<int64_t>(static_cast<uint32_t>(loc) / static_cast<uint32_t>(page_size))
                           : loc / page_size;
  if (page >= num_pages) return;
  const int64_t in_page = loc - page * page_size;
  uint8_t* pg = cache + page * bpp;
  uint8_t* row = pg + in_page * kPackRowBytes;
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
  if (lane >= kPackNope / 8) {  // rope: the bf16 bytes verbatim
    uint8_t* dst = row + kPackNope + 16 * (lane - kPackNope / 8);
    if (kVec) {
      *reinterpret_cast<uint4*>(dst) = w;
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) dst[i] = static_cast<uint8_t>(ww[i / 4] >> (8 * (i % 4)));
    }
  }
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(ww[i] << 16);
    v[2 * i + 1] = __uint_as_float(ww[i] & 0xffff0000u);
  }
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(v[i]));
  // max over the tile's 8 lanes (DPP within aligned groups of 8)
  mx = fmaxf(mx, __uint_as_float(lane_xor<1>(__float_as_uint(mx), lane)));
  mx = fmaxf(mx, __uint_as_float(lane_xor<2>(__float_as_uint(mx), lane)));
  mx = fmaxf(mx, __uint_as_float(lane_xor<4>(__float_as_uint(mx), lane)));
  if (lane >= kPackNope / 8) return;
  const float r = fmaxf(mx, 1e-8f) / 448.0f;
  const int E = ceil_log2(r);
  const float inv = __builtin_ldexpf(1.0f, -E);  // exact: E in [-35, 121] for bf16 inputs
  float qv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) qv[i] = fminf(fmaxf(v[i] * inv, -448.0f), 448.0f);
  const uint32_t b[2] = {e4m3fn_rne4(qv[0], qv[1], qv[2], qv[3]), e4m3fn_rne4(qv[4], qv[5], qv[6], qv[7])};
  uint8_t* dst = row + 8 * lane;
  if (kVec) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(b[0], b[1]);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = static_cast<uint8_t>(b[i / 4] >> (8 * (i % 4)));
  }
  if ((lane & 7) == 0) {
    const int byte = E + 127;
    pg[static_cast<int64_t>(page_size) * kPackRowBytes + in_page * kPackScaleBytes + (lane >> 3)] =
        static_cast<uint8_t>(byte < 0 ? 0 : (byte > 255 ? 255 : byte));
  }
}

// Each wavefront packs kPackTokensPerWave consecutive tokens.  Their slots and
// their 1 KiB rows are requested as one batch before any is processed (tokens
// past the end re-read the last token and are skipped), so a wavefront waits
// for one memory round trip, not for a slot and then its token.
template <bool kVec>
__global__ __launch_bounds__(kPackWaves * kWave) void dsv4_pack_kernel(const uint16_t* __restrict__ tokens,
                                                                       const int32_t* __restrict__ locs,
                                                                       int64_t num_tokens, uint8_t* __restrict__ cache,
                                                                       int64_t num_pages, int64_t bpp,
                                                                       int page_size) {
  const int lane = threadIdx.x % kWave;
  const int64_t t0 = (static_cast<int64_t>(blockIdx.x) * kPackWaves + threadIdx.x / kWave) * kPackTokensPerWave;
  if (t0 >= num_tokens) return;
  int32_t loc_raw[kPackTokensPerWave];
  uint4 w[kPackTokensPerWave];
#pragma unroll
  for (int i = 0; i < kPackTokensPerWave; ++i) {
    const int64_t t = t0 + i < num_tokens ? t0 + i : num_tokens - 1;
    const uint16_t* src = tokens + t * 512;
    // with no slot list the slot load re-reads the token and is dropped
    loc_raw[i] = load_global_i32(locs ? static_cast<const void*>(locs + t) : static_cast<const void*>(src));
    w[i] = load_global_u4(src + 8 * lane);
  }
  // Consumed here, before any branch, so no load is sunk under one.
#pragma unroll
  for (int i = 0; i < kPackTokensPerWave; ++i)
    asm volatile("" : "+v"(w[i].x), "+v"(w[i].y), "+v"(w[i].z), "+v"(w[i].w), "+v"(loc_raw[i]));
#pragma unroll
  for (int i = 0; i < kPackTokensPerWave; ++i) {
    const int64_t t = t0 + i;
    if (t < num_tokens)
      pack_token<kVec>(w[i], locs ? static_cast<int64_t>(loc_raw[i]) : t, lane, cache, num_pages, bpp, page_size);
  }
}

}  // namespace
}  // namespace csahca

using namespace csahca;

extern "C" int csahca_dsv4_pack_tokens(const void* k_tokens, const int32_t* locs, int64_t num_tokens,
                                       uint8_t* cache, int64_t num_pages, int64_t bytes_per_page,
                                       int64_t page_size, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(num_tokens >= 0 && num_pages >= 0 && bytes_per_page >= 0, "negative dimension");
  CSAHCA_REQUIRE(page_size > 0 && page_size <= INT_MAX, "page_size must be positive");
  CSAHCA_REQUIRE(bytes_per_page >= page_size * (kPackRowBytes + kPackScaleBytes),
                 "bytes_per_page is too small for DSV4 page layout");
  if (num_tokens == 0 || num_pages == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(k_tokens && cache, "null tensor pointer");
  CSAHCA_REQUIRE(reinterpret_cast<uintptr_t>(k_tokens) % 16 == 0, "k_tokens must be 16-byte aligned");
  const int64_t blocks = ceil_div(num_tokens, kPackWaves * kPackTokensPerWave);
  CSAHCA_REQUIRE(blocks <= INT32_MAX, "too many tokens in one call");
  const bool vec = reinterpret_cast<uintptr_t>(cache) % 16 == 0 && bytes_per_page % 16 == 0;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const dim3 grid(static_cast<uint32_t>(blocks));
  const uint16_t* tp = static_cast<const uint16_t*>(k_tokens);
  return vec ? launch("dsv4_pack_kernel", dsv4_pack_kernel<true>, grid, dim3(kPackWaves * kWave), 0, stream, tp,
                      locs, num_tokens, cache, num_pages, bytes_per_page, static_cast<int>(page_size))
             : launch("dsv4_pack_kernel", dsv4_pack_kernel<false>, grid, dim3(kPackWaves * kWave), 0, stream, tp,
                      locs, num_tokens, cache, num_pages, bytes_per_page, static_cast<int>(page_size));
}
