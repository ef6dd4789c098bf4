// dsv4.hip -- DSV4 MQA decode over the paged FP8 latent cache, for gfx950.
//
// Cache layout (hybrid_attention/dsv4_correctness.py:10-21,
// csrc/dsv4_attention.cu:13-19): page p at byte p*bpp; page_size token rows of
// 576 bytes (448 OCP e4m3 "nope" + 64 bf16 "rope"), then page_size scale rows
// of 8 bytes (7 UE8M0 exponents: nope value = e4m3 * 2^(byte-127)).
//
// Kernel design: the latent row of a slot is shared by every query head (MQA,
// V = K).  A work item is one wavefront over (query, group of HG heads, tile
// of slots): it fetches each slot's row ONCE (lanes 0..55 take 8 fp8 bytes +
// their tile's scale byte, lanes 56..63 take 16 bytes of rope), dequantises
// into 8 fp32 registers per lane, and updates the online softmax of all HG
// heads from those registers.  Partials (m, l, acc[512]) per (query, head,
// tile) are merged by dsv4_merge_kernel, which also folds the attention sink
// in as a virtual token of logit `sink` and value 0.
#include "common.hpp"

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <type_traits>

namespace csahca {
namespace {

constexpr int kNope = 448;
constexpr int kRope = 64;
constexpr int kDim = kNope + kRope;
constexpr int kRowBytes = kNope + 2 * kRope;  // 576
constexpr int kScaleTiles = kNope / 64;       // 7
constexpr int kScaleBytes = kScaleTiles + 1;  // 8
constexpr int kHeadGroup = 8;                 // heads per work item

// OCP e4m3fn byte -> fp32 from the format definition (bias 7; exponent field 0
// is subnormal m * 2^-9; S.1111.111 is NaN).
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t e = (b >> 3) & 15u;
  const uint32_t m = b & 7u;
  float mag = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : static_cast<float>(m) * 0x1p-9f;
  mag = ((b & 0x7fu) == 0x7fu) ? __builtin_nanf("") : mag;
  return (b & 0x80u) ? -mag : mag;
}

// UE8M0 exponent byte -> 2^(byte-127).
__device__ __forceinline__ float ue8m0_to_f32(uint32_t s) {
  return s ? __uint_as_float(s << 23) : 0x1p-127f;
}

// Resolve slot s of a query to a row pointer (nullptr if the slot is skipped).
struct CacheView {
  const uint8_t* base;
  int64_t num_pages;
  int64_t bpp;
  int page_size;
  int page_shift;  // log2(page_size) when it is a power of two, else -1
};

CacheView cache_view(const void* base, int64_t num_pages, int64_t bpp, int64_t page_size) {
  int shift = -1;
  if (page_size > 0 && (page_size & (page_size - 1)) == 0) {
    shift = 0;
    while ((int64_t{1} << shift) < page_size) ++shift;
  }
  return CacheView{static_cast<const uint8_t*>(base), num_pages, bpp, static_cast<int>(page_size), shift};
}

__device__ __forceinline__ const uint8_t* row_ptr(const CacheView& c, int32_t loc,
                                                  const uint8_t** scale_row) {
  if (loc < 0) return nullptr;
  // A shift for power-of-two pages: an integer division would sit between the
  // slot index load and the row load it addresses.
  const int64_t page = c.page_shift >= 0 ? (loc >> c.page_shift) : loc / c.page_size;
  if (page >= c.num_pages) return nullptr;
  const int64_t in_page = loc - page * c.page_size;
  const uint8_t* pg = c.base + page * c.bpp;
  *scale_row = pg + static_cast<int64_t>(c.page_size) * kRowBytes + in_page * kScaleBytes;
  return pg + in_page * kRowBytes;
}

// Dequantise this lane's 8 columns of a token row (columns 8*lane .. 8*lane+7).
template <bool kVec>
__device__ __forceinline__ void load_row8(const uint8_t* __restrict__ row,
                                          const uint8_t* __restrict__ srow, int lane, float* kv) {
  if (lane < kNope / 8) {
    const float s = ue8m0_to_f32(srow[lane >> 3]);
    uint32_t lo, hi;
    if (kVec) {
      const uint2 w = *reinterpret_cast<const uint2*>(row + 8 * lane);
      lo = w.x;
      hi = w.y;
    } else {
      const uint8_t* p = row + 8 * lane;
      lo = p[0] | (p[1] << 8) | (p[2] << 16) | (static_cast<uint32_t>(p[3]) << 24);
      hi = p[4] | (p[5] << 8) | (p[6] << 16) | (static_cast<uint32_t>(p[7]) << 24);
    }
    // v_cvt_pk_f32_fp8 decodes OCP e4m3fn exactly (all 256 codes checked on
    // the device); the products with 2^(b-127) are exact in fp32.
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t p0 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(lo), false);
    const f32x2_t p1 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(lo), true);
    const f32x2_t p2 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(hi), false);
    const f32x2_t p3 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(hi), true);
    kv[0] = p0[0] * s;
    kv[1] = p0[1] * s;
    kv[2] = p1[0] * s;
    kv[3] = p1[1] * s;
    kv[4] = p2[0] * s;
    kv[5] = p2[1] * s;
    kv[6] = p3[0] * s;
    kv[7] = p3[1] * s;
  } else {
    const uint8_t* p = row + kNope + 16 * (lane - kNope / 8);
    uint32_t w[4];
    if (kVec) {
      const uint4 v = *reinterpret_cast<const uint4*>(p);
      w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = p[4 * i] | (p[4 * i + 1] << 8) | (p[4 * i + 2] << 16) |
               (static_cast<uint32_t>(p[4 * i + 3]) << 24);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv[2 * i] = __uint_as_float(w[i] << 16);
      kv[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

// One slot's share of a lane as raw words, requested unconditionally by every
// lane (16-byte aligned rows): the 8 nope bytes at 8*lane (for lanes 56..63
// these are rope bytes 448..511, inside the row), the lane's 16 rope bytes
// (nope lanes re-read the first rope block) and the tile's scale byte (lanes
// 56..63 read the slot's pad byte).  The lane's part is selected after the
// loads, so a batch of slots is one memory round trip.
struct RawRow8 {
  uint2 nope;
  uint4 rope;
  uint32_t scale;
};

__device__ __forceinline__ RawRow8 load_raw_row8(const uint8_t* row, const uint8_t* srow, int lane) {
  const bool nope = lane < kNope / 8;
  RawRow8 r;
  r.nope = load_global_u2(row + 8 * lane);
  r.rope = load_global_u4(row + kNope + 16 * (nope ? 0 : lane - kNope / 8));
  r.scale = load_global_raw<uint8_t>(srow + (lane >> 3));
  return r;
}

__device__ __forceinline__ void decode_raw_row8(const RawRow8& r, int lane, float* kv) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  const float s = ue8m0_to_f32(r.scale);
  const f32x2_t p0 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(r.nope.x), false);
  const f32x2_t p1 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(r.nope.x), true);
  const f32x2_t p2 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(r.nope.y), false);
  const f32x2_t p3 = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(r.nope.y), true);
  const float fp8v[8] = {p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
  const uint32_t w[4] = {r.rope.x, r.rope.y, r.rope.z, r.rope.w};
  const bool nope = lane < kNope / 8;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float lo = __uint_as_float(w[i] << 16), hi = __uint_as_float(w[i] & 0xffff0000u);
    kv[2 * i] = nope ? fp8v[2 * i] * s : lo;
    kv[2 * i + 1] = nope ? fp8v[2 * i + 1] * s : hi;
  }
}

// Eight consecutive elements of T at p (aligned to 8 * sizeof(T)) widened to
// fp32, through 1, 2 or 4 unconditional 16-byte loads.
template <typename T>
__device__ __forceinline__ void load8_f32(const T* p, float* out) {
  constexpr int N = Vec16<T>::N;
#pragma unroll
  for (int i = 0; i < 8 / N; ++i) widen16<T>(load_global_u4(p + N * i), out + N * i);
}

struct Dsv4Args {
  CacheView swa;
  CacheView extra;
  const int32_t* idx;
  const int32_t* lens;
  const int32_t* eidx;
  const int32_t* elens;
  float* part_ml;
  float* part_acc;
  int heads;
  int head_groups;
  int topk_slots;
  int extra_slots;  // 0 when there is no extra cache
  int tile;
  int num_tiles;
  float qscale;  // softmax_scale * log2(e)
};

// 64-bit value of lane l (l uniform across the wavefront).
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), l));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v >> 32), l));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// One halving step of a wavefront reduce-scatter over N per-lane partial sums:
// lanes with bit D set keep the upper half of the values, the others the lower
// half; each lane sends the half it drops to lane ^ D and adds what it gets.
template <int D, int N>
__device__ __forceinline__ void rs_half(float* v, int lane) {
  const bool upper = (lane & D) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float keep = upper ? v[i + N / 2] : v[i];
    const float send = upper ? v[i] : v[i + N / 2];
    v[i] = keep + __uint_as_float(lane_xor<D>(__float_as_uint(send), lane));
  }
}

// Reduce-scatter of 32 per-lane partial sums (31 lane moves instead of the
// 192 of 32 butterfly all-reduces): lane L ends with the wavefront total of
// v[L >> 1].
__device__ __forceinline__ float wave_reduce_scatter32(float* v, int lane) {
  rs_half<32, 32>(v, lane);
  rs_half<16, 16>(v, lane);
  rs_half<8, 8>(v, lane);
  rs_half<4, 4>(v, lane);
  rs_half<2, 2>(v, lane);
  return v[0] + __uint_as_float(lane_xor<1>(__float_as_uint(v[0]), lane));
}

// Slots per batch of row loads: kSlotBatch x kHeadGroup = 32 dot products per
// reduce-scatter.
constexpr int kSlotBatch = 4;
static_assert(kSlotBatch * kHeadGroup == 32, "one reduce-scatter of 32 sums per batch");

template <typename T, bool kVec>
__global__ __launch_bounds__(64) void dsv4_tile_kernel(const T* __restrict__ q, Dsv4Args a) {
  const int lane = threadIdx.x;
  // 32-bit index arithmetic (the grid is < 2^32 blocks).
  const uint32_t item = blockIdx.x;
  const int t = static_cast<int>(item % static_cast<uint32_t>(a.num_tiles));
  const uint32_t rest = item / static_cast<uint32_t>(a.num_tiles);
  const int hg = static_cast<int>(rest % static_cast<uint32_t>(a.head_groups));
  const int64_t query = rest / static_cast<uint32_t>(a.head_groups);
  const int h0 = hg * kHeadGroup;
  const int nh = min(kHeadGroup, a.heads - h0);

  float qr[kHeadGroup][8];
  int n_swa, n_extra;
  if constexpr (kVec) {
    // One batch: both lengths (a missing list reads q and is dropped) and the
    // q rows of the group (heads past the last re-read head h0, then zeroed).
    const int32_t len_raw = load_global_i32(a.lens ? static_cast<const void*>(a.lens + query)
                                                   : static_cast<const void*>(q));
    const int32_t elen_raw = load_global_i32(a.elens ? static_cast<const void*>(a.elens + query)
                                                     : static_cast<const void*>(q));
#pragma unroll
    for (int h = 0; h < kHeadGroup; ++h)
      load8_f32<T>(q + ((query * a.heads) + h0 + (h < nh ? h : 0)) * kDim + 8 * lane, qr[h]);
#pragma unroll
    for (int h = 0; h < kHeadGroup; ++h)
#pragma unroll
      for (int e = 0; e < 8; ++e) qr[h][e] = h < nh ? qr[h][e] * a.qscale : 0.f;
    n_swa = a.lens ? max(0, min(len_raw, a.topk_slots)) : a.topk_slots;
    n_extra = a.extra_slots > 0 ? (a.elens ? max(0, min(elen_raw, a.extra_slots)) : a.extra_slots) : 0;
  } else {
#pragma unroll
    for (int h = 0; h < kHeadGroup; ++h) {
      if (h < nh) {
        const T* qp = q + ((query * a.heads) + h0 + h) * kDim + 8 * lane;
#pragma unroll
        for (int e = 0; e < 8; ++e) qr[h][e] = to_f32(qp[e]) * a.qscale;
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) qr[h][e] = 0.f;
      }
    }
    n_swa = a.lens ? max(0, min(a.lens[query], a.topk_slots)) : a.topk_slots;
    n_extra = a.extra_slots > 0 ? (a.elens ? max(0, min(a.elens[query], a.extra_slots)) : a.extra_slots) : 0;
  }
  const int total = a.topk_slots + a.extra_slots;
  const int s0 = t * a.tile;
  const int s1 = min(s0 + a.tile, total);

  float m[kHeadGroup], l[kHeadGroup], acc[kHeadGroup][8];
#pragma unroll
  for (int h = 0; h < kHeadGroup; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[h][e] = 0.f;
  }

  for (int g = s0; g < s1; g += kWave) {
    // Lane j resolves slot g + j (index load + page math) for the whole group.
    const int s = g + lane;
    const uint8_t* rp = nullptr;
    const uint8_t* sp = nullptr;
    if constexpr (kVec) {
      // The slot's index is requested unconditionally (lanes past the tile
      // re-read its last slot) and the slot dropped after the load.
      const int sc = s < s1 ? s : s1 - 1;
      const bool in_swa = sc < a.topk_slots;
      const int32_t* ip = in_swa ? a.idx + query * a.topk_slots + sc
                                 : a.eidx + query * a.extra_slots + (sc - a.topk_slots);
      const int32_t loc = load_global_i32(ip);
      const bool live = s < s1 && (in_swa ? s < n_swa : s - a.topk_slots < n_extra);
      const uint8_t* sp_c = nullptr;
      const uint8_t* rp_c = row_ptr(in_swa ? a.swa : a.extra, loc, &sp_c);
      rp = live ? rp_c : nullptr;
      sp = live ? sp_c : nullptr;
    } else if (s < s1) {
      if (s < a.topk_slots) {
        if (s < n_swa) rp = row_ptr(a.swa, a.idx[query * a.topk_slots + s], &sp);
      } else {
        const int j = s - a.topk_slots;
        if (j < n_extra) rp = row_ptr(a.extra, a.eidx[query * a.extra_slots + j], &sp);
      }
    }
    const unsigned long long valid = __ballot(rp != nullptr);
    if (valid == 0ull) continue;
    // Skipped slots fetch the first valid slot's row (in bounds); their scores are masked.
    const int first = __ffsll(static_cast<long long>(valid)) - 1;
    const uint64_t r_first = readlane64(reinterpret_cast<uint64_t>(rp), first);
    const uint64_t s_first = readlane64(reinterpret_cast<uint64_t>(sp), first);
    const uint64_t r_lane = rp ? reinterpret_cast<uint64_t>(rp) : r_first;
    const uint64_t s_lane = rp ? reinterpret_cast<uint64_t>(sp) : s_first;
    const int cnt = min(kWave, s1 - g);
    for (int b = 0; b < cnt; b += kSlotBatch) {
      const uint32_t ok = static_cast<uint32_t>(valid >> b) & ((1u << kSlotBatch) - 1u);
      if (ok == 0u) continue;
      float kv[kSlotBatch][8];
      if constexpr (kVec) {
        RawRow8 raw[kSlotBatch];
#pragma unroll
        for (int j = 0; j < kSlotBatch; ++j) {
          const uint8_t* row = reinterpret_cast<const uint8_t*>(readlane64(r_lane, b + j));
          const uint8_t* srow = reinterpret_cast<const uint8_t*>(readlane64(s_lane, b + j));
          raw[j] = load_raw_row8(row, srow, lane);
        }
        // No decoding is scheduled between the loads (it would wait for the
        // first slot before the others are requested).
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kSlotBatch; ++j) decode_raw_row8(raw[j], lane, kv[j]);
      } else {
#pragma unroll
        for (int j = 0; j < kSlotBatch; ++j) {
          const uint8_t* row = reinterpret_cast<const uint8_t*>(readlane64(r_lane, b + j));
          const uint8_t* srow = reinterpret_cast<const uint8_t*>(readlane64(s_lane, b + j));
          load_row8<kVec>(row, srow, lane, kv[j]);
        }
      }
      float part[kSlotBatch * kHeadGroup];
#pragma unroll
      for (int j = 0; j < kSlotBatch; ++j)
#pragma unroll
        for (int h = 0; h < kHeadGroup; ++h) {
          float d = 0.f;
#pragma unroll
          for (int e = 0; e < 8; ++e) d = fmaf(qr[h][e], kv[j][e], d);
          part[j * kHeadGroup + h] = d;
        }
      const float tot = wave_reduce_scatter32(part, lane);
#pragma unroll
      for (int h = 0; h < kHeadGroup; ++h) {
        float sc[kSlotBatch];
        float mb = -INFINITY;
#pragma unroll
        for (int j = 0; j < kSlotBatch; ++j) {
          const float x =
              __int_as_float(__builtin_amdgcn_readlane(__float_as_int(tot), 2 * (j * kHeadGroup + h)));
          sc[j] = ((ok >> j) & 1u) ? x : -INFINITY;
          mb = fmaxf(mb, sc[j]);
        }
        const float m_new = fmaxf(m[h], mb);  // finite: the batch has a valid slot
        const float alpha = fast_exp2(m[h] - m_new);
        float p[kSlotBatch];
        float psum = 0.f;
#pragma unroll
        for (int j = 0; j < kSlotBatch; ++j) {
          p[j] = fast_exp2(sc[j] - m_new);
          psum += p[j];
        }
        l[h] = l[h] * alpha + psum;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float x = acc[h][e] * alpha;
#pragma unroll
          for (int j = 0; j < kSlotBatch; ++j) x = fmaf(p[j], kv[j][e], x);
          acc[h][e] = x;
        }
        m[h] = m_new;
      }
    }
  }

#pragma unroll
  for (int h = 0; h < kHeadGroup; ++h) {
    if (h < nh) {
      const int64_t p = ((query * a.heads) + h0 + h) * a.num_tiles + t;
      float* dst = a.part_acc + p * kDim + 8 * lane;
      *reinterpret_cast<float4*>(dst) = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[h][4], acc[h][5], acc[h][6], acc[h][7]);
      if (lane == 0) {
        a.part_ml[2 * p] = m[h];
        a.part_ml[2 * p + 1] = l[h];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Grouped-head MFMA path (bf16 queries): one workgroup = (query, 16 heads,
// split of the slot list), tiles of 32 slots.  QK^T and PV are real
// contractions here (16 heads share each latent row), so they run on
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation:
//   * the 4 wavefronts split the 512-dim contraction of QK^T (wave w owns
//     dims [128w, 128w+128)); lane l loads 8 consecutive latent bytes of slot
//     l%16 (+16) -- exactly the MFMA B layout -- dequantises them in registers
//     (e4m3 x 2^(b-127), rounded to bf16 as the reference dequant does) and
//     also stores them, 16 bytes per lane, into a row-major [slot][dim] V
//     tile in LDS;
//   * the 4 partial score blocks meet in LDS; every wavefront computes the
//     same online-softmax update, whose probabilities already sit in the MFMA
//     A layout of PV (lane l: head l%16, slots 8(l/16)..+7);
//   * wave w accumulates O[16 heads][128w .. 128w+127] over the tiles; its PV
//     B operands come out of the row-major V tile already transposed, via the
//     gfx950 LDS transpose read ds_read_b64_tr_b16.
// Output: (m, l, acc[512]) partials per (query, head, split), merged with the
// sink by dsv4_merge_kernel.
// MFMA lane layout (16x16x32 bf16): A lane l elem j = A[l%16][8(l/16)+j];
// B lane l elem j = B[8(l/16)+j][l%16]; C lane l elem i = C[4(l/16)+i][l%16].
// ds_read_b64_tr_b16 (probed on the device): within each 16-lane group, with
// local lane a passing the address of 4 consecutive 16-bit values E[a][0..3],
// local lane i receives elem j = E[4j + i/4][i%4].  Passing &V[8g + a/4][n0 +
// 4(a%4)] in group g therefore hands lane i the values V[8g + j][n0 + i],
// j = 0..3: half of the PV B operand (the other half starts 4 rows lower).
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMfmaHeads = 16;
constexpr int kMfmaSlots = 32;
// Row stride of the LDS V tile in bf16: 1072 B = 268 dwords (12 mod 64 banks).
// The 16 lanes of a 16-byte row store (slots 0..15) then start 12 banks apart
// mod 64 (distinct 4-bank groups), and the 4 row groups of a transpose read
// (rows r..r+3, 8 dwords each) land on banks [0,8), [12,20), [24,32), [36,44):
// both conflict-free.
constexpr int kVRowStride = kDim + 24;
// Row stride of the per-wave score partials in floats (36 = 4 mod 32): the
// stores of the 4 lane groups (rows 4 apart) and the 16-byte reads (rows
// l%16) both spread over all banks.
constexpr int kSpStride = kMfmaSlots + 4;
constexpr int kMfmaWaves = 4;
constexpr int kMfmaThreads = kMfmaWaves * kWave;
constexpr int kKStepsPerWave = kDim / 32 / kMfmaWaves;  // 4 k-steps of 32 dims
constexpr int kNopeSteps = kNope / 32;                  // k-steps 0..13 are e4m3, 14..15 bf16 rope
constexpr int kOutTiles = kDim / kMfmaWaves / 16;       // 8 blocks of 16 output dims per wave

// 8 e4m3 bytes x 2^(b-127) -> 8 bf16, packed two per word.  The gfx950 scaled
// conversion gives exactly round_bf16(e4m3 * 2^(b-127)) for scale bytes
// 0..254 (all 256 codes checked on the device); byte 255 (fp32 scale 2^128 =
// inf in the reference's arithmetic) takes the software decode.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t bf16x2_bits(bf16x2_t v) { return __builtin_bit_cast(uint32_t, v); }

__device__ __forceinline__ uint4 dequant8_bf16_hw(uint2 w, uint32_t sbyte) {
  const float s = ue8m0_to_f32(sbyte);
  return make_uint4(bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, s, false)),
                    bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, s, true)),
                    bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, s, false)),
                    bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, s, true)));
}

// True when one of the 7 scale bytes of a token (bytes 0..6 of w) is 255.
// Bytes equal to 255 become 0 in the complements; the pad byte 7 is cleared
// first, so its complement is 0xff and never counts.
__device__ __forceinline__ bool has_scale_255(uint2 w) {
  const uint32_t a = ~w.x, b = ~(w.y & 0x00ffffffu);
  return (((a - 0x01010101u) & ~a) | ((b - 0x01010101u) & ~b)) & 0x80808080u;
}

// The software decode alone (for sub-tiles that hold a scale byte of 255).
__device__ __forceinline__ uint4 dequant8_bf16_sw(uint2 w, uint32_t sbyte) {
  const float s = ue8m0_to_f32(sbyte);
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t word = i < 2 ? w.x : w.y;
    const uint32_t b0 = (word >> (16 * (i & 1))) & 0xffu;
    const uint32_t b1 = (word >> (16 * (i & 1) + 8)) & 0xffu;
    o[i] = static_cast<uint32_t>(float_to_bf16_bits(e4m3_to_f32(b0) * s)) |
           (static_cast<uint32_t>(float_to_bf16_bits(e4m3_to_f32(b1) * s)) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ uint4 dequant8_bf16(uint2 w, uint32_t sbyte) {
  if (sbyte != 255u) {
    const float s = ue8m0_to_f32(sbyte);
    return make_uint4(bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, s, false)),
                      bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, s, true)),
                      bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, s, false)),
                      bf16x2_bits(__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, s, true)));
  }
  const float s = ue8m0_to_f32(sbyte);
  uint32_t o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t word = i < 2 ? w.x : w.y;
    const uint32_t b0 = (word >> (16 * (i & 1))) & 0xffu;
    const uint32_t b1 = (word >> (16 * (i & 1) + 8)) & 0xffu;
    o[i] = static_cast<uint32_t>(float_to_bf16_bits(e4m3_to_f32(b0) * s)) |
           (static_cast<uint32_t>(float_to_bf16_bits(e4m3_to_f32(b1) * s)) << 16);
  }
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// How a (query, head group, split) workgroup finishes.
enum MfmaOut : int {
  kMfmaPartials = 0,  // write (m, l, acc) partials for dsv4_merge_kernel
  kMfmaDirect = 1,    // the only split: merge with the sink and write the output
};

struct MfmaArgs {
  int splits;           // slot-list splits per (query, head group)
  int tiles_per_split;  // 32-slot tiles per split
  int mfma_groups;      // head groups of 16
  const float* sink;    // kMfmaDirect
  bf16* out;
};

template <int kOut>
__global__ __launch_bounds__(kMfmaThreads) void dsv4_mfma_kernel(const bf16* __restrict__ q, Dsv4Args a,
                                                                 MfmaArgs m) {
  __shared__ __align__(16) uint16_t vtile[kMfmaSlots * kVRowStride];     // [slot][dim] bf16 bits
  __shared__ __align__(16) float sp[kMfmaWaves][kMfmaHeads][kSpStride];   // per-wave score partials
  __shared__ float xch[kMfmaWaves][kMfmaHeads];                           // per-wave head exchange

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform: branches on it stay scalar
  const int lane = tid % kWave;
  const int grp = lane / 16;  // lane group (MFMA k / row block)
  const int l16 = lane % 16;
  // 32-bit index arithmetic (the grid is < 2^32 blocks): 64-bit divisions are
  // long scalar sequences on the critical path.
  const uint32_t item = blockIdx.x;
  const int split = static_cast<int>(item % static_cast<uint32_t>(m.splits));
  const uint32_t rest = item / static_cast<uint32_t>(m.splits);
  const int hg = static_cast<int>(rest % static_cast<uint32_t>(m.mfma_groups));
  const int64_t query = rest / static_cast<uint32_t>(m.mfma_groups);
  const int h0 = hg * kMfmaHeads;
  const int nh = min(kMfmaHeads, a.heads - h0);

  // Q A-operands of this wave's k-steps: head h0 + l16, dims 32 kk + 8 grp .. +7.
  // Prologue loads are unconditional (a head past nh re-reads head h0, a
  // missing length array reads q) and consumed after all are issued, so the
  // q operands, the lengths and the first slot indices are one batch.
  uint4 qw[kKStepsPerWave];
  const int hq = h0 + min(l16, nh - 1);
#pragma unroll
  for (int i = 0; i < kKStepsPerWave; ++i) {
    const int d0 = 32 * (wave * kKStepsPerWave + i) + 8 * grp;
    qw[i] = load_global_u4(q + ((query * a.heads) + hq) * kDim + d0);
  }
  const int32_t len_raw = load_global_i32(a.lens ? static_cast<const void*>(a.lens + query) : static_cast<const void*>(q));
  const int32_t elen_raw =
      load_global_i32(a.elens ? static_cast<const void*>(a.elens + query) : static_cast<const void*>(q));
  bf16x8_t qa[kKStepsPerWave];
#pragma unroll
  for (int i = 0; i < kKStepsPerWave; ++i)
    qa[i] = __builtin_bit_cast(bf16x8_t, l16 < nh ? qw[i] : make_uint4(0u, 0u, 0u, 0u));

  const int n_swa = a.lens ? max(0, min(len_raw, a.topk_slots)) : a.topk_slots;
  const int n_extra = a.extra_slots > 0 ? (a.elens ? max(0, min(elen_raw, a.extra_slots)) : a.extra_slots) : 0;
  const int total = a.topk_slots + a.extra_slots;
  const int t0 = split * m.tiles_per_split;
  const int t1 = min(t0 + m.tiles_per_split, (total + kMfmaSlots - 1) / kMfmaSlots);

  float mh = -INFINITY, lh = 0.f;  // softmax state of head l16 (identical in every lane group)
  f32x4_t o[kOutTiles];
#pragma unroll
  for (int j = 0; j < kOutTiles; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // A skipped slot reads this workgroup's own q row instead (always in bounds,
  // 1 KiB >= one 584-byte latent row + scales) and its bytes are zeroed after
  // the load, so every load is unconditional (see slot_loc).
  const uint8_t* dummy = reinterpret_cast<const uint8_t*>(q + (query * a.heads + h0) * kDim);
  // Token location of slot l16 + 16 nt of tile t, or -1 when skipped.  The
  // index loads are unconditional (clamped positions, results selected after
  // the load): loads under per-lane branches make the compiler wait for every
  // outstanding load at the join, which would serialise the prefetch below.
  // Issue (two index loads) and resolve (validity select) are separate steps
  // so a caller can issue several slots' loads before consuming any.
  struct SlotIdx {
    int32_t li, le;
  };
  auto slot_issue = [&](int t, int nt) -> SlotIdx {
    const int s = t * kMfmaSlots + l16 + 16 * nt;
    const int32_t* ip = a.topk_slots > 0 ? a.idx + query * a.topk_slots + min(s, a.topk_slots - 1)
                                         : reinterpret_cast<const int32_t*>(dummy);
    const int32_t* ep = a.extra_slots > 0
                            ? a.eidx + query * a.extra_slots + min(max(s - a.topk_slots, 0), a.extra_slots - 1)
                            : reinterpret_cast<const int32_t*>(dummy);
    return SlotIdx{load_global_i32(ip), load_global_i32(ep)};
  };
  auto slot_resolve = [&](int t, int nt, SlotIdx r) -> int32_t {
    const int s = t * kMfmaSlots + l16 + 16 * nt;
    const bool in_swa = s < a.topk_slots;
    const bool valid = t < t1 && s < total && (in_swa ? s < n_swa : s - a.topk_slots < n_extra);
    return valid ? (in_swa ? r.li : r.le) : -1;
  };
  auto slot_loc = [&](int t, int nt) -> int32_t { return slot_resolve(t, nt, slot_issue(t, nt)); };
  // This lane's latent bytes of a tile: for each slot, the wave's 4 k-steps
  // (8 e4m3 bytes in .x/.y, or 16 bytes of bf16 rope) and the scale row.
  struct Rows {
    uint4 raw[2][kKStepsPerWave];  // as loaded (a skipped slot's bytes are masked at use)
    uint2 sc8[2];
    uint32_t valid;  // tile-wide slot mask (ballot)
    uint32_t ok;     // this lane's slots: bit nt
  };
  auto issue_rows = [&](int t, const int32_t* loc, Rows& r) {
    const uint8_t* rp[2];
    const uint8_t* srp[2];
    bool ok[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const int s = t * kMfmaSlots + l16 + 16 * nt;
      const uint8_t* sr = nullptr;
      const uint8_t* rr = loc[nt] >= 0 ? row_ptr(s < a.topk_slots ? a.swa : a.extra, loc[nt], &sr) : nullptr;
      ok[nt] = rr != nullptr;
      rp[nt] = ok[nt] ? rr : dummy;
      srp[nt] = ok[nt] ? sr : dummy;
    }
    r.valid = static_cast<uint32_t>(__ballot(ok[0]) & 0xffffull) |
              (static_cast<uint32_t>(__ballot(ok[1]) & 0xffffull) << 16);
    r.ok = (ok[0] ? 1u : 0u) | (ok[1] ? 2u : 0u);
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      r.sc8[nt] = load_global_u2(srp[nt]);
#pragma unroll
      for (int i = 0; i < kKStepsPerWave; ++i) {
        const int kk = wave * kKStepsPerWave + i;
        const int d0 = 32 * kk + 8 * grp;
        // 16 bytes either way: e4m3 bytes d0.. (the first 8 are used; the rest
        // stay inside the 576-byte row) or bf16 rope values d0-448..
        const int off = kk < kNopeSteps ? d0 : kNope + 2 * (d0 - kNope);
        r.raw[nt][i] = load_global_u4(rp[nt] + off);
      }
    }
  };

  // Two-stage pipeline: while tile t is processed, the rows of tile t+1 and
  // the slot locations of tile t+2 are in flight (lds_barrier keeps them so).
  Rows cur, nxt;
  // Prologue: the index loads of tiles t0 and t0+1 go out with the q and
  // length loads above; the empty asm makes every one of them issue before
  // any is consumed.
  SlotIdx i00 = slot_issue(t0, 0), i01 = slot_issue(t0, 1), i10 = slot_issue(t0 + 1, 0),
          i11 = slot_issue(t0 + 1, 1);
  asm volatile("" : "+v"(i00.li), "+v"(i00.le), "+v"(i01.li), "+v"(i01.le), "+v"(i10.li), "+v"(i10.le),
               "+v"(i11.li), "+v"(i11.le));
  int32_t loc[2] = {slot_resolve(t0, 0, i00), slot_resolve(t0, 1, i01)};
  issue_rows(t0, loc, cur);
  int32_t loc_n[2] = {slot_resolve(t0 + 1, 0, i10), slot_resolve(t0 + 1, 1, i11)};
  for (int t = t0; t < t1; ++t) {
    if (t + 1 < t1) issue_rows(t + 1, loc_n, nxt);
    const int32_t loc_nn[2] = {slot_loc(t + 2, 0), slot_loc(t + 2, 1)};
    const uint32_t valid = cur.valid;  // same mask in every wavefront: workgroup-uniform
    if (valid != 0u) {
      // Dequantise, store V^T, and accumulate this wave's share of QK^T.
      // Scale byte 255 (fp32 scale 2^128) needs the software decode: decided
      // once per tile for the whole wavefront, so the common path has no
      // per-lane branch.
      const bool any255 =
          __ballot(((cur.ok & 1u) && has_scale_255(cur.sc8[0])) || ((cur.ok & 2u) && has_scale_255(cur.sc8[1]))) != 0ull;
      f32x4_t sacc[2];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        sacc[nt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        const int slot = l16 + 16 * nt;
#pragma unroll
        for (int i = 0; i < kKStepsPerWave; ++i) {
          const int kk = wave * kKStepsPerWave + i;
          const int d0 = 32 * kk + 8 * grp;
          uint4 kb;
          if (kk < kNopeSteps) {
            const int blk = kk / 2;
            const uint32_t sbyte = (blk < 4 ? cur.sc8[nt].x >> (8 * blk) : cur.sc8[nt].y >> (8 * (blk - 4))) & 0xffu;
            const uint2 bytes = make_uint2(cur.raw[nt][i].x, cur.raw[nt][i].y);
            kb = any255 ? dequant8_bf16(bytes, sbyte) : dequant8_bf16_hw(bytes, sbyte);
          } else {
            kb = cur.raw[nt][i];
          }
          if (!((cur.ok >> nt) & 1u)) kb = make_uint4(0u, 0u, 0u, 0u);  // skipped slot: zero K and V
          // V row: this lane's 8 dims of its slot, as they are.
          *reinterpret_cast<uint4*>(&vtile[slot * kVRowStride + d0]) = kb;
          sacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[i], __builtin_bit_cast(bf16x8_t, kb), sacc[nt],
                                                             0, 0, 0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) sp[wave][4 * grp + e][slot] = sacc[nt][e];
      }
      lds_barrier();

      // Scores of head l16, slots 8 grp .. 8 grp + 7 (the PV A layout).
      float x[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = 0.f;
#pragma unroll
      for (int w = 0; w < kMfmaWaves; ++w) {
        const float4 u = *reinterpret_cast<const float4*>(&sp[w][l16][8 * grp]);
        const float4 v = *reinterpret_cast<const float4*>(&sp[w][l16][8 * grp + 4]);
        x[0] += u.x; x[1] += u.y; x[2] += u.z; x[3] += u.w;
        x[4] += v.x; x[5] += v.y; x[6] += v.z; x[7] += v.w;
      }
      float mb = -INFINITY;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        x[j] = ((valid >> (8 * grp + j)) & 1u) ? x[j] * a.qscale : -INFINITY;
        mb = fmaxf(mb, x[j]);
      }
      mb = fmaxf(mb, __uint_as_float(lane_xor<16>(__float_as_uint(mb), lane)));
      mb = fmaxf(mb, __uint_as_float(lane_xor<32>(__float_as_uint(mb), lane)));
      const float m_new = fmaxf(mh, mb);  // finite: the tile has a valid slot
      const float alpha = fast_exp2(mh - m_new);
      float ps = 0.f;
      uint32_t pw[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const float p0 = fast_exp2(x[j] - m_new), p1 = fast_exp2(x[j + 1] - m_new);
        ps += p0 + p1;
        pw[j / 2] = static_cast<uint32_t>(float_to_bf16_bits(p0)) |
                    (static_cast<uint32_t>(float_to_bf16_bits(p1)) << 16);
      }
      ps += __uint_as_float(lane_xor<16>(__float_as_uint(ps), lane));
      ps += __uint_as_float(lane_xor<32>(__float_as_uint(ps), lane));
      lh = lh * alpha + ps;
      mh = m_new;
      // alpha per output row (head 4 grp + e of the C layout) through LDS.
      if (lane < kMfmaHeads) xch[wave][lane] = alpha;
      wave_lds_sync();
      float ar[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) ar[e] = xch[wave][4 * grp + e];
      const bf16x8_t pa = __builtin_bit_cast(bf16x8_t, make_uint4(pw[0], pw[1], pw[2], pw[3]));
      // PV B operand of output block j (dims n0 = 128 wave + 16 j): lane l
      // needs V[8 grp + 0..7][n0 + l16], read transposed from the row-major
      // tile (local lane a passes &V[8 grp + a/4 (+4)][n0 + 4 (a%4)]).
      typedef short i16x4_t __attribute__((ext_vector_type(4)));
      typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;
      const uint16_t* vsrc = &vtile[(8 * grp + l16 / 4) * kVRowStride + wave * (kDim / kMfmaWaves) + 4 * (l16 % 4)];
#pragma unroll
      for (int j = 0; j < kOutTiles; ++j) {
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vsrc + 16 * j));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vsrc + 4 * kVRowStride + 16 * j));
        const u32x2_t lw = __builtin_bit_cast(u32x2_t, lo), hw = __builtin_bit_cast(u32x2_t, hi);
        const uint4 vb = make_uint4(lw[0], lw[1], hw[0], hw[1]);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[j][e] *= ar[e];
        o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, __builtin_bit_cast(bf16x8_t, vb), o[j], 0, 0, 0);
      }
      lds_barrier();  // vtile / sp are rewritten by the next tile
    }
    cur = nxt;
    loc_n[0] = loc_nn[0];
    loc_n[1] = loc_nn[1];
  }

  if constexpr (kOut == kMfmaPartials) {
    // Partials: m, l of head l16 (wave 0, lane group 0), acc rows of the C layout.
    const int64_t pbase = (query * a.heads + h0) * m.splits + split;  // + h * splits
    if (wave == 0 && lane < nh) {
      const int64_t pi = pbase + static_cast<int64_t>(lane) * m.splits;
      a.part_ml[2 * pi] = mh;
      a.part_ml[2 * pi + 1] = lh;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int h = 4 * grp + e;
      if (h < nh) {
        float* dst = a.part_acc + (pbase + static_cast<int64_t>(h) * m.splits) * kDim + wave * (kDim / kMfmaWaves) + l16;
#pragma unroll
        for (int j = 0; j < kOutTiles; ++j) dst[16 * j] = o[j][e];
      }
    }
    return;
  }

  const int dcol = wave * (kDim / kMfmaWaves) + l16;  // this lane's output dims: dcol + 16 j
  if constexpr (kOut == kMfmaDirect) {
    // The merge of dsv4_merge_kernel over one partial (the sink a virtual token
    // of logit sink[h] and value 0; the same operations).  Rows 4 grp + e of
    // the C layout: their m, l sit in lanes 4 grp + e.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int h = 4 * grp + e;
      const float me = __shfl(mh, h), le = __shfl(lh, h);
      if (h >= nh) continue;
      const float sk = m.sink ? m.sink[h0 + h] * kLog2e : -INFINITY;
      const float mx = le > 0.f ? fmaxf(sk, me) : sk;
      const bool use = mx != -INFINITY && le > 0.f;
      const float w = use ? fast_exp2(me - mx) : 0.f;
      float L = use ? fmaf(le, w, 0.f) : 0.f;
      if (m.sink && mx != -INFINITY) L += fast_exp2(sk - mx);
      const float inv = le != le ? __builtin_nanf("") : (L > 0.f ? 1.f / L : 0.f);
      bf16* orow = m.out + (query * a.heads + h0 + h) * kDim + dcol;
#pragma unroll
      for (int j = 0; j < kOutTiles; ++j) orow[16 * j] = from_f32<bf16>((use ? fmaf(w, o[j][e], 0.f) : 0.f) * inv);
    }
    return;
  }
}

// ---------------------------------------------------------------------------
// Per-query grouped-head kernel (bf16 queries, automatic tiling): one
// workgroup = (query, 16 heads) and the query's WHOLE slot list, so each
// latent row is fetched once per workgroup, the split partials never leave
// the CU and there is no merge launch.  Head groups of one query are blocks
// b, b + 8, b + 16, ... -- the same XCD (blocks go to XCD blockIdx % 8), so
// at H = 64 the four workgroups that read a query's rows share one L2.
//
// The slot list goes in rounds of W sub-tiles of 16 slots (W = 4 or 8
// wavefronts; wavefront w takes sub-tile w of each round).  Per round each
// wavefront
//   * loads its sub-tile's 16 rows (lane l: slot l%16, 16-byte chunks l/16 +
//     4i of the 576-byte row, and the slot's 8 scale bytes), dequantises the
//     e4m3 part to bf16 exactly as the reference dequant rounds it, and stores
//     the [slot][dim] tile in its own LDS slice;
//   * computes S^T = K Q^T on v_mfma_f32_16x16x32_bf16 (A = the tile row of
//     slot l%16, B = the query rows, both read from LDS 16 bytes at a time):
//     lane l holds S^T[slot 4(l/16)+e][head l%16], and publishes the masked,
//     scaled scores in LDS;
//   * after a barrier, runs the online softmax of head l%16 over the round's
//     W sub-tiles (its 4 slots of each and the 3 lanes with the same l%16, row
//     swaps 16 and 32) -- every wavefront the same, so m and l agree -- with
//     the bf16-rounded probabilities as the B operand of the PV product;
//   * accumulates O^T = V^T P^T on v_mfma_f32_16x16x16_bf16 for ITS 512 / W
//     output dims (blocks of 16) over all W tiles; the A operand V^T[dim][slot
//     4g..4g+3] comes straight out of the row-major tiles through
//     ds_read_b64_tr_b16.  Lane l holds O^T[dim 16 blk + 4(l/16) + e][head
//     l%16], so the softmax rescale of a lane is its own head's factor.
// Finally each wavefront normalises its dims with the sink as a virtual token
// of logit sink[h] and value 0 (csrc/dsv4_attention.cu:252-269) and stores
// them: no partials to merge.
// MFMA lane layouts: 16x16x32 as above; 16x16x16: A lane l elem j =
// A[l%16][4(l/16)+j], B lane l elem j = B[4(l/16)+j][l%16], C as 16x16x32.
// ---------------------------------------------------------------------------
// Two floats to packed bf16 with gfx950's packed conversion (one
// v_cvt_pk_bf16_f32, no branch between the MFMAs whose operands it forms):
// round to nearest even, infinities unchanged, NaN quietened -- the bits of
// float_to_bf16_bits for every one of the 2^32 fp32 inputs (compared
// exhaustively on the device), so the results are those of the software
// rounding it replaces.
__device__ __forceinline__ uint32_t bf16x2_nb(float lo, float hi) {
  typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
  const bf16x2_v v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

constexpr int kQSub = 16;                 // slots per sub-tile
constexpr int kQHeads = 16;
// LDS tile row: 536 bf16 = 1072 B = 67 16-byte units = 268 dwords (12 mod 64
// banks).  The dequant's 16-byte stores (16 lanes: slots 0..15 of one column)
// and the 16-byte A reads (slot l%16) step 3 units per slot, a permutation of
// the 16 units of the 64 banks; the 4 rows of a transpose read (8 bytes x 4
// lanes each) land on banks [0,8), [12,20), [24,32), [36,44): all
// conflict-free.
constexpr int kQRow = kDim + 24;
constexpr int kQTileBytes = kQSub * kQRow * 2;
// Query rows in LDS (the B operand of S^T, shared by the wavefronts): 520
// bf16 = 1040 B = 260 dwords (4 mod 64 banks), so the 16 heads' 16-byte reads
// of one lane group cover the 64 banks once.
constexpr int kQQRow = kDim + 8;
constexpr int kQBuf = 2;                  // sub-tiles of rows in flight per wavefront
constexpr int kQNopeChunks = kNope / 16;  // 28 chunks of 16 e4m3 bytes
constexpr int kQChunksPerLane = 9;        // 7 e4m3 chunks + 2 rope chunks

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

struct QueryArgs {
  int64_t nq;
  int groups;         // head groups of 16
  int nsub;           // 16-slot sub-tiles of the slot list
  const float* sink;  // [heads] or null
  bf16* out;
};

// One sub-tile of a lane's row data, as loaded.
struct QRows {
  uint4 c[kQChunksPerLane];
  uint2 sc;
  bool ok;
};

// DS: workgroups per (query, 16 heads), each writing kDim / DS of the output
// dims (every one of them dequantises and scores the whole slot list; the
// PV products are split).  The DS workgroups of a query share its XCD.
template <int W, int DS = 1>
__global__ __launch_bounds__(W * kWave) void dsv4_query_kernel(const bf16* __restrict__ q, Dsv4Args a, QueryArgs g) {
  constexpr int NT = W * kWave;
  constexpr int DW = kDim / DS;                         // output dims of this workgroup
  constexpr int QOB = DW / W / 16;                      // 16-dim output blocks per wavefront
  constexpr int QQU = kQHeads * (kDim / 8) / NT;       // 16-byte query units per thread
  // The W tiles, then each wavefront's masked scores (a lane's 4 floats) and
  // its sub-tile's slot bits.
  constexpr int QSM = W * kQTileBytes + W * kWave * 4 * 4 + W * 4;
  static_assert(QSM + kQHeads * kQQRow * 2 <= 160 * 1024, "LDS of one workgroup");
  __shared__ __align__(16) uint8_t smem[QSM];
  __shared__ __align__(16) uint16_t qlds[kQHeads * kQQRow];

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int grp = lane / 16;
  const int l16 = lane % 16;
  const uint32_t blk = blockIdx.x;
  const uint32_t r = blk / 8;
  const uint32_t gx = static_cast<uint32_t>(g.groups) * DS;  // (head group, dim part) pairs of a query
  const uint32_t hgx = r % gx;
  const int hg = static_cast<int>(hgx / DS);
  const int part = static_cast<int>(hgx % DS);
  const int64_t query = static_cast<int64_t>(r / gx) * 8 + blk % 8;
  if (query >= g.nq) return;
  const int h0 = hg * kQHeads;
  const int nh = min(kQHeads, a.heads - h0);

  // Prologue batch: the query rows (B operand of S^T: head h0 + l16, dims
  // 32 kk + 8 grp .. +7; heads past nh re-read head h0 + nh - 1 and are
  // zeroed), the lengths and the sink -- unconditional loads, consumed later.
  const void* anyp = static_cast<const void*>(q);
  const int32_t len_raw = load_global_i32(a.lens ? static_cast<const void*>(a.lens + query) : anyp);
  const int32_t elen_raw = load_global_i32(a.elens ? static_cast<const void*>(a.elens + query) : anyp);

  const int total = a.topk_slots + a.extra_slots;
  const uint8_t* dummy = reinterpret_cast<const uint8_t*>(q + (query * a.heads + h0) * kDim);  // >= 1 KiB, in bounds
  // Slot index of sub-tile t for this lane (slot 16 t + l16): both index
  // loads are unconditional (clamped positions), the choice comes later.
  struct SlotIdx {
    int32_t li, le;
  };
  auto idx_issue = [&](int t) -> SlotIdx {
    const int s = t * kQSub + l16;
    const int32_t* ip = a.topk_slots > 0 ? a.idx + query * a.topk_slots + min(s, a.topk_slots - 1)
                                         : reinterpret_cast<const int32_t*>(dummy);
    const int32_t* ep = a.extra_slots > 0
                            ? a.eidx + query * a.extra_slots + min(max(s - a.topk_slots, 0), a.extra_slots - 1)
                            : reinterpret_cast<const int32_t*>(dummy);
    return SlotIdx{load_global_i32(ip), load_global_i32(ep)};
  };
  int n_swa = 0, n_extra = 0;  // set once the length loads are consumed
  auto rows_issue = [&](int t, SlotIdx si, QRows& rw) {
    const int s = t * kQSub + l16;
    const bool in_swa = s < a.topk_slots;
    const bool valid = s < total && (in_swa ? s < n_swa : s - a.topk_slots < n_extra);
    const int32_t loc = valid ? (in_swa ? si.li : si.le) : -1;
    const uint8_t* sr = nullptr;
    const uint8_t* rr = loc >= 0 ? row_ptr(in_swa ? a.swa : a.extra, loc, &sr) : nullptr;
    rw.ok = rr != nullptr;
    const uint8_t* rp = rw.ok ? rr : dummy;
    const uint8_t* sp = rw.ok ? sr : dummy;
#pragma unroll
    for (int i = 0; i < 7; ++i) rw.c[i] = load_global_u4(rp + 16 * (grp + 4 * i));
#pragma unroll
    for (int i = 0; i < 2; ++i) rw.c[7 + i] = load_global_u4(rp + kNope + 16 * (grp + 4 * i));
    rw.sc = load_global_u2(sp);
  };

  const int nsub_w = g.nsub > wave ? (g.nsub - wave + W - 1) / W : 0;  // this wave's sub-tiles
  static_assert(kQBuf == 2, "two row buffers below");
  const int last_sub = max(g.nsub - 1, 0);
  SlotIdx si0 = idx_issue(min(wave, last_sub)), si1 = idx_issue(min(wave + W, last_sub));
  // The query rows and the sink go out after the lengths and the first
  // indices, so waiting for those (the rows' addresses) does not wait for them.
  // Thread t loads the workgroup's 16-byte query units t + 64 W u (head e / 64,
  // dims 8 (e % 64) .. +7; heads past nh re-read head h0 + nh - 1 and are
  // stored as zeros), staged once in LDS for all the wavefronts.
  uint4 qw[QQU];
#pragma unroll
  for (int u = 0; u < QQU; ++u) {
    const int e = tid + NT * u;
    qw[u] = load_global_u4(q + (query * a.heads + h0 + min(e / (kDim / 8), nh - 1)) * kDim + 8 * (e % (kDim / 8)));
  }
  const int hq = h0 + min(l16, nh - 1);
  const float sink_raw = g.sink ? load_global_raw<float>(g.sink + hq) : -INFINITY;
  asm volatile("" : "+v"(si0.li), "+v"(si0.le), "+v"(si1.li), "+v"(si1.le));
  n_swa = a.lens ? max(0, min(len_raw, a.topk_slots)) : a.topk_slots;
  n_extra = a.extra_slots > 0 ? (a.elens ? max(0, min(elen_raw, a.extra_slots)) : a.extra_slots) : 0;
  // Sub-tile t of this wave is global sub-tile wave + 4 t; past the list a
  // buffer is loaded from the dummy row with no valid slot.
  auto sub_of = [&](int t) { return t < nsub_w ? wave + W * t : g.nsub; };
  QRows cur, nxt;  // rows of this wave's sub-tiles t and t + 1
  rows_issue(sub_of(0), si0, cur);
  rows_issue(sub_of(1), si1, nxt);
  SlotIdx sn = idx_issue(min(wave + W * kQBuf, last_sub));  // indices of sub-tile kQBuf
#pragma unroll
  for (int u = 0; u < QQU; ++u) {
    const int e = tid + NT * u;
    *reinterpret_cast<uint4*>(qlds + (e / (kDim / 8)) * kQQRow + 8 * (e % (kDim / 8))) =
        e / (kDim / 8) < nh ? qw[u] : make_uint4(0u, 0u, 0u, 0u);
  }
  lds_barrier();  // every wavefront's query units are in LDS before the first sub-tile
  const uint16_t* qrow = qlds + l16 * kQQRow + 8 * grp;  // B operand: head l16, dims 32 kk + 8 grp ..

  uint16_t* tile = reinterpret_cast<uint16_t*>(smem + wave * kQTileBytes);
  float* xs = reinterpret_cast<float*>(smem + W * kQTileBytes);  // [wave][lane][4] masked scores
  uint32_t* flags = reinterpret_cast<uint32_t*>(xs + W * kWave * 4);  // [wave] valid-slot bits
  float m = -INFINITY, l = 0.f;  // online softmax of head l16 (this lane's 4 slots of each sub-tile)
  f32x4_t o[QOB];
#pragma unroll
  for (int j = 0; j < QOB; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // V^T A operand of output block j (dims 128 wave + 16 j ..) of a tile: lane a
  // of group g passes &V[4g + a/4][128 wave + 16 j + 4(a%4)].
  const int vofs = (4 * grp + l16 / 4) * kQRow + 4 * (l16 % 4) + DW * part + (DW / W) * wave;

  // This wavefront's sub-tile of the round: dequantise it into its tile, score
  // it against the 16 heads, publish the masked scores and the slot bits.
  auto score_own = [&](const QRows& rw, bool has) {
    const uint32_t valid16 = has ? static_cast<uint32_t>(__ballot(rw.ok) & 0xffffull) : 0u;  // wave-uniform
    if (lane == 0) flags[wave] = valid16;
    if (valid16 == 0u) return;
    // Scale byte 255 takes the software decode, decided once per sub-tile.
    const bool any255 = __ballot(rw.ok && has_scale_255(rw.sc)) != 0ull;
    uint16_t* trow = tile + l16 * kQRow;
    if (!any255) {
#pragma unroll
      for (int i = 0; i < 7; ++i) {
        const uint32_t sbyte = (i < 4 ? rw.sc.x >> (8 * i) : rw.sc.y >> (8 * (i - 4))) & 0xffu;
        uint4 lo = dequant8_bf16_hw(make_uint2(rw.c[i].x, rw.c[i].y), sbyte);
        uint4 hi = dequant8_bf16_hw(make_uint2(rw.c[i].z, rw.c[i].w), sbyte);
        if (!rw.ok) lo = hi = make_uint4(0u, 0u, 0u, 0u);  // skipped slot: zero K and V
        const int c = grp + 4 * i;
        *reinterpret_cast<uint4*>(trow + 16 * c) = lo;
        *reinterpret_cast<uint4*>(trow + 16 * c + 8) = hi;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 7; ++i) {  // rare (a scale byte of 255): the software decode
        const uint32_t sbyte = (i < 4 ? rw.sc.x >> (8 * i) : rw.sc.y >> (8 * (i - 4))) & 0xffu;
        uint4 lo = dequant8_bf16_sw(make_uint2(rw.c[i].x, rw.c[i].y), sbyte);
        uint4 hi = dequant8_bf16_sw(make_uint2(rw.c[i].z, rw.c[i].w), sbyte);
        if (!rw.ok) lo = hi = make_uint4(0u, 0u, 0u, 0u);
        const int c = grp + 4 * i;
        *reinterpret_cast<uint4*>(trow + 16 * c) = lo;
        *reinterpret_cast<uint4*>(trow + 16 * c + 8) = hi;
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
      *reinterpret_cast<uint4*>(trow + kNope + 8 * (grp + 4 * i)) = rw.ok ? rw.c[7 + i] : make_uint4(0u, 0u, 0u, 0u);
    wave_lds_sync();
    // The A reads (tile rows) and B reads (query rows) go out 8 at a time
    // ahead of their MFMAs (one LDS round trip per 8, not per MFMA); two
    // accumulators halve the dependent MFMA chain.
    f32x4_t sacc0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, sacc1 = sacc0;
#pragma unroll
    for (int k0 = 0; k0 < 16; k0 += 8) {
      uint4 kr[8], qr[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) kr[u] = *reinterpret_cast<const uint4*>(trow + 32 * (k0 + u) + 8 * grp);
#pragma unroll
      for (int u = 0; u < 8; ++u) qr[u] = *reinterpret_cast<const uint4*>(qrow + 32 * (k0 + u));
#pragma unroll
      for (int u = 0; u < 8; u += 2) {
        sacc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[u]),
                                                        __builtin_bit_cast(bf16x8_t, qr[u]), sacc0, 0, 0, 0);
        sacc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[u + 1]),
                                                        __builtin_bit_cast(bf16x8_t, qr[u + 1]), sacc1, 0, 0, 0);
      }
    }
    f32x4_t x;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      x[e] = ((valid16 >> (4 * grp + e)) & 1u) ? (sacc0[e] + sacc1[e]) * a.qscale : -INFINITY;
    *reinterpret_cast<f32x4_t*>(xs + (wave * kWave + lane) * 4) = x;
  };

  // Rounds of W sub-tiles (wavefront w's sub-tile of round r is W r + w).
  // Every wavefront runs the same online softmax over the round's 16 W slots --
  // the same scores in the same order, so the same m and l everywhere -- and
  // accumulates O^T for its own 512 / W output dims from all W tiles: no partials
  // to merge at the end.  Sub-tiles with no valid slot take no part.
  const int rounds = (g.nsub + W - 1) / W;
  for (int rd = 0; rd < rounds; ++rd) {
    score_own(cur, rd < nsub_w);
    cur = nxt;
    if (rd + kQBuf < nsub_w) {
      rows_issue(sub_of(rd + kQBuf), sn, nxt);
      sn = idx_issue(min(wave + W * (rd + kQBuf + 1), last_sub));
    }
    lds_barrier();  // the round's tiles, scores and slot bits are in LDS
    uint32_t fl[W];
    uint32_t any = 0u;
#pragma unroll
    for (int u = 0; u < W; ++u) {
      fl[u] = flags[u];
      any |= fl[u];
    }
    if (any != 0u) {  // workgroup-uniform
      float xr[W][4];
      float mt = -INFINITY;
#pragma unroll
      for (int u = 0; u < W; ++u) {
        const f32x4_t v = fl[u] ? *reinterpret_cast<const f32x4_t*>(xs + (u * kWave + lane) * 4)
                                : f32x4_t{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xr[u][e] = v[e];
          mt = fmaxf(mt, v[e]);
        }
      }
      mt = fmaxf(mt, __uint_as_float(lane_xor<16>(__float_as_uint(mt), lane)));
      mt = fmaxf(mt, __uint_as_float(lane_xor<32>(__float_as_uint(mt), lane)));
      // Lazy rescale: the running max m only moves when a score exceeds it by
      // more than 2^8 (so probabilities stay below 2^8, exact enough in fp32
      // and as bf16 PV operands) or on the first round with a valid slot; the
      // output accumulators are rescaled only when some head of the wavefront
      // moved.
      const bool move = mt > m + 8.f;  // m = -inf: always
      const float m_new = move ? mt : m;
      const float alpha = move ? fast_exp2(m - m_new) : 1.f;
      float ps = 0.f;
      i16x4_t pb[W];
#pragma unroll
      for (int u = 0; u < W; ++u) {
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[e] = fast_exp2(xr[u][e] - m_new);
          ps += p[e];
        }
        // an empty sub-tile's probabilities are zero (its scores are -inf)
        pb[u] = __builtin_bit_cast(i16x4_t, make_uint2(bf16x2_nb(p[0], p[1]), bf16x2_nb(p[2], p[3])));
      }
      l = l * alpha + ps;
      m = m_new;
      if (__any(move)) {
#pragma unroll
        for (int j = 0; j < QOB; ++j)
#pragma unroll
          for (int e = 0; e < 4; ++e) o[j][e] *= alpha;
      }
      // An empty sub-tile (no tile written this round) reads the first valid
      // tile's rows against its zero probabilities: no branch around the
      // MFMAs (a branch there moves the accumulators out of the registers
      // the MFMAs keep them in, and back, for every tile).
      int first = W - 1;
#pragma unroll
      for (int u = W - 1; u >= 0; --u) first = fl[u] ? u : first;
#pragma unroll
      for (int u = 0; u < W; ++u) {
        const uint16_t* vsrc = reinterpret_cast<const uint16_t*>(smem + (fl[u] ? u : first) * kQTileBytes) + vofs;
        i16x4_t vt[QOB];
#pragma unroll
        for (int j = 0; j < QOB; ++j)
          vt[j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vsrc + 16 * j));
#pragma unroll
        for (int j = 0; j < QOB; ++j)
          o[j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt[j], pb[u], o[j], 0, 0, 0);
      }
    }
    lds_barrier();  // the tiles and scores are rewritten by the next round
  }
  l += __uint_as_float(lane_xor<16>(__float_as_uint(l), lane));
  l += __uint_as_float(lane_xor<32>(__float_as_uint(l), lane));

  // Normalise with the sink as a virtual token of logit sink[h] and value 0
  // (csrc/dsv4_attention.cu:252-269): M = max(sink, m), L = l 2^(m - M) +
  // 2^(sink - M), out = O 2^(m - M) / L; a NaN score makes the head NaN, as
  // torch.softmax does in the oracle.
  const float sk = g.sink ? sink_raw * kLog2e : -INFINITY;
  const float mx = l > 0.f ? fmaxf(sk, m) : sk;
  const float w = (l > 0.f && mx != -INFINITY) ? fast_exp2(m - mx) : 0.f;
  float L = w * (l > 0.f ? l : 0.f);
  if (g.sink && mx != -INFINITY) L += fast_exp2(sk - mx);
  const float sc = l != l ? __builtin_nanf("") : (L > 0.f ? w / L : 0.f);
  if (l16 < nh) {
    bf16* orow = g.out + (query * a.heads + h0 + l16) * kDim + DW * part + (DW / W) * wave + 4 * grp;
#pragma unroll
    for (int j = 0; j < QOB; ++j) {
      *reinterpret_cast<uint2*>(orow + 16 * j) =
          make_uint2(bf16x2_nb(o[j][0] * sc, o[j][1] * sc), bf16x2_nb(o[j][2] * sc, o[j][3] * sc));
    }
  }
}

// ---------------------------------------------------------------------------
// One-pass grouped-head kernel (dsv4_onepass_kernel<NW, SUBS, DS>): slot
// lists of at most NW * SUBS * 16 slots.  A workgroup of NW wavefronts is one
// (query, 16 heads, dim part), as for dsv4_query_kernel, but nothing runs in
// rounds:
//   1. every lane requests the indices of its SUBS slots, the lengths, the
//      query rows (staged in LDS) and the sink; then, as soon as the indices
//      arrive, the latent rows of its sub-tiles -- wavefront w owns sub-tiles
//      w, w + NW, ... of 16 slots, so the whole slot list is in flight after
//      two dependent round trips;
//   2. each wavefront reads its B operand of S^T = K Q^T (the 16 query rows)
//      from LDS into registers once, then per sub-tile dequantises the rows
//      straight into MFMA A operands -- the contraction runs over the dims in
//      the order of the 16-byte row chunks a lane holds (chunk c = grp + 4 i
//      of e4m3 gives the k-steps 2 i and 2 i + 1, rope chunk grp + 4 i the
//      k-step 14 + i), and the query operand is read in the same order -- and
//      writes the values of this workgroup's output dims to a row-major V
//      tile in LDS;
//   3. one exact softmax per head over the whole list: per-wavefront maxima
//      through LDS, then p = 2^(s - M) (fp32 sums, bf16 operands for PV)
//      written as P^T rows in LDS;
//   4. O^T = V^T P^T on v_mfma_f32_16x16x16_bf16 for the workgroup's 16-dim
//      output blocks (dealt to the wavefronts round-robin) over all sub-tiles
//      (V^T through ds_read_b64_tr_b16), and the sink as a virtual token of
//      logit sink[h] and value 0 (csrc/dsv4_attention.cu:252-269).
// Two shapes: 12 wavefronts with one sub-tile each (lists of up to 192 slots:
// every wavefront's QK is one sub-tile, so no wavefront serialises two; the
// query staging has LDS of its own) and 8 wavefronts with two each (up to
// 256; the V tiles then take the staging's LDS once the operand is read).
// Scores, probabilities and sums are those of the other MFMA kernels up to
// fp32 summation order (the softmax subtracts the exact maximum).  Each output
// block's MFMA chain is the same in every shape and dim-part count; the
// softmax sum adds per-wavefront partial sums, so the two shapes can differ in
// its last bits.
// A zero latent row (and scale bytes) for the slots of the one-pass kernel
// that are past their list's length or invalid: they load it in place of a
// cache row, so their K and V values are exact zeros with no per-value select
// (e4m3 0 at scale byte 0 is +0, the rope bf16 0 is +0); their scores are
// masked to -inf all the same.
__device__ __align__(16) uint8_t g_dsv4_zero_row[1024];

constexpr int kOpMaxSlots = 256;  // the largest list of the one-pass shapes
constexpr int kOpProw = 272;      // P^T row stride in bf16 (136 dwords = 8 mod 64 banks)

template <int NW, int SUBS, int DS>
struct OnePassLayout {
  static constexpr int SLOTS = NW * SUBS * kQSub;          // capacity
  static constexpr int DW = kDim / DS;                     // output dims of a workgroup
  static constexpr int VROW = DW + 24;                     // V tile row in bf16 (dwords = 12 mod 64)
  static constexpr int NB = DW / 16;                       // 16-dim output blocks of the workgroup
  static constexpr int OB = (NB + NW - 1) / NW;            // blocks per wavefront (at most)
  static constexpr int TILE_BYTES = SLOTS * VROW * 2;
  static constexpr int Q_BYTES = kQHeads * kQQRow * 2;     // query staging
  static constexpr int SMALL = NW * 16 * 4 * 2 + kQHeads * kOpProw * 2;  // maxima, sums, P^T
  static constexpr bool ALIAS = TILE_BYTES + Q_BYTES + SMALL > 160 * 1024;  // staging inside the V tiles
  static constexpr int QS = ALIAS ? 0 : TILE_BYTES;        // query staging offset
  static constexpr int R0 = ALIAS ? (TILE_BYTES > Q_BYTES ? TILE_BYTES : Q_BYTES) : TILE_BYTES + Q_BYTES;
  static constexpr int MX = R0;                            // [waves][16] maxima
  static constexpr int LS = MX + NW * 16 * 4;              // [waves][16] sums
  static constexpr int PT = LS + NW * 16 * 4;              // [16 heads][kOpProw] bf16
  static constexpr int BYTES = PT + kQHeads * kOpProw * 2;
  static_assert(SLOTS <= kOpMaxSlots, "P^T rows hold kOpMaxSlots slots");
  static_assert(BYTES <= 160 * 1024, "LDS of one workgroup");
};

template <int NW, int SUBS, int DS>
__global__ __launch_bounds__(NW * kWave) void dsv4_onepass_kernel(const int32_t* idx, const int32_t* eidx,
                                                                   const int32_t* lens, const int32_t* elens,
                                                                   int32_t topk_slots, int32_t extra_slots,
                                                                   int32_t groups, int32_t nq, int32_t heads,
                                                                   const bf16* __restrict__ q, Dsv4Args a,
                                                                   QueryArgs g) {
  // The leading scalars repeat what the slot-index loads need (the library
  // preloads them into SGPRs at wave launch); the copies in a and g are the
  // same values.
  a.idx = idx;
  a.eidx = eidx;
  a.lens = lens;
  a.elens = elens;
  a.topk_slots = topk_slots;
  a.extra_slots = extra_slots;
  a.heads = heads;
  g.groups = groups;
  g.nq = nq;
  using Lay = OnePassLayout<NW, SUBS, DS>;
  constexpr int NT = NW * kWave;
  constexpr int DW = Lay::DW, VROW = Lay::VROW, NB = Lay::NB, OB = Lay::OB;
  constexpr int QUNITS = kQHeads * (kDim / 8);              // 16-byte query units of the workgroup
  constexpr int QQU = (QUNITS + NT - 1) / NT;               // per thread
  __shared__ __align__(16) uint8_t smem[Lay::BYTES];
  uint16_t* vtile = reinterpret_cast<uint16_t*>(smem);
  uint16_t* qlds = reinterpret_cast<uint16_t*>(smem + Lay::QS);
  float* mxs = reinterpret_cast<float*>(smem + Lay::MX);
  float* lss = reinterpret_cast<float*>(smem + Lay::LS);
  uint16_t* pt = reinterpret_cast<uint16_t*>(smem + Lay::PT);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int lane = tid % kWave;
  const int grp = lane / 16;
  const int l16 = lane % 16;
  const uint32_t blk = blockIdx.x;
  const uint32_t r = blk / 8;
  const uint32_t gx = static_cast<uint32_t>(g.groups) * DS;
  const uint32_t hgx = r % gx;
  const int hg = static_cast<int>(hgx / DS);
  const int part = static_cast<int>(hgx % DS);
  const int64_t query = static_cast<int64_t>(r / gx) * 8 + blk % 8;
  if (query >= g.nq) return;
  const int h0 = hg * kQHeads;
  const int nh = min(kQHeads, a.heads - h0);
  const int nsub = g.nsub;
  const int total = a.topk_slots + a.extra_slots;

  // ---- 1. indices, lengths, query rows, sink; then the rows -----------------
  // The index and length loads need only the preloaded arguments: an absent
  // list or length reads the query's first index of the other list instead
  // (the list is never empty here), not the query rows.
  const int32_t* anyi = a.topk_slots > 0 ? a.idx + query * a.topk_slots : a.eidx + query * a.extra_slots;
  const void* anyp = static_cast<const void*>(anyi);
  const int32_t len_raw = load_global_i32(a.lens ? static_cast<const void*>(a.lens + query) : anyp);
  const int32_t elen_raw = load_global_i32(a.elens ? static_cast<const void*>(a.elens + query) : anyp);
  int32_t li[SUBS], le[SUBS];
#pragma unroll
  for (int j = 0; j < SUBS; ++j) {
    const int s = (wave + NW * j) * kQSub + l16;
    const int32_t* ip = a.topk_slots > 0 ? a.idx + query * a.topk_slots + min(s, a.topk_slots - 1) : anyi;
    const int32_t* ep =
        a.extra_slots > 0 ? a.eidx + query * a.extra_slots + min(max(s - a.topk_slots, 0), a.extra_slots - 1) : anyi;
    li[j] = load_global_i32(ip);
    le[j] = load_global_i32(ep);
  }
  uint4 qw[QQU];
#pragma unroll
  for (int u = 0; u < QQU; ++u) {
    const int e = min(tid + NT * u, QUNITS - 1);  // (units past the last re-read it; not stored)
    qw[u] = load_global_u4(q + (query * a.heads + h0 + min(e / (kDim / 8), nh - 1)) * kDim + 8 * (e % (kDim / 8)));
  }
  // (unconditional: a load under a branch would make the wait-count pass wait
  // for every load in flight at the join)
  const float sink_raw = load_global_raw<float>(g.sink ? static_cast<const void*>(g.sink + h0 + min(l16, nh - 1))
                                                       : anyp);
  // The rows of invalid slots read the zero row.
  const uint8_t* dummy = g_dsv4_zero_row;
  // The cache views the row addresses need, requested now, while the slot
  // indices are in flight (left to itself the compiler loads them where the
  // addresses are formed: one more dependent round trip after the indices).
  asm volatile("" ::"s"(a.swa.base), "s"(a.swa.num_pages), "s"(a.swa.bpp), "s"(a.swa.page_size),
               "s"(a.swa.page_shift), "s"(a.extra.base), "s"(a.extra.num_pages), "s"(a.extra.bpp),
               "s"(a.extra.page_size), "s"(a.extra.page_shift));
#pragma unroll
  for (int j = 0; j < SUBS; ++j) asm volatile("" : "+v"(li[j]), "+v"(le[j]));
  const int n_swa = a.lens ? max(0, min(len_raw, a.topk_slots)) : a.topk_slots;
  const int n_extra = a.extra_slots > 0 ? (a.elens ? max(0, min(elen_raw, a.extra_slots)) : a.extra_slots) : 0;
  QRows rw[SUBS];
#pragma unroll
  for (int j = 0; j < SUBS; ++j) {
    const int s = (wave + NW * j) * kQSub + l16;
    const bool in_swa = s < a.topk_slots;
    const bool valid = s < total && (in_swa ? s < n_swa : s - a.topk_slots < n_extra);
    const int32_t loc = valid ? (in_swa ? li[j] : le[j]) : -1;
    const uint8_t* sr = nullptr;
    const uint8_t* rr = loc >= 0 ? row_ptr(in_swa ? a.swa : a.extra, loc, &sr) : nullptr;
    rw[j].ok = rr != nullptr;
    const uint8_t* rp = rw[j].ok ? rr : dummy;
    const uint8_t* sp = rw[j].ok ? sr : dummy;
#pragma unroll
    for (int i = 0; i < 7; ++i) rw[j].c[i] = load_global_u4(rp + 16 * (grp + 4 * i));
#pragma unroll
    for (int i = 0; i < 2; ++i) rw[j].c[7 + i] = load_global_u4(rp + kNope + 16 * (grp + 4 * i));
    rw[j].sc = load_global_u2(sp);
  }

  // ---- 2. query operand into registers; per sub-tile dequant, V tile, QK ----
#pragma unroll
  for (int u = 0; u < QQU; ++u) {
    const int e = tid + NT * u;
    if (e < QUNITS)
      *reinterpret_cast<uint4*>(qlds + (e / (kDim / 8)) * kQQRow + 8 * (e % (kDim / 8))) =
          e / (kDim / 8) < nh ? qw[u] : make_uint4(0u, 0u, 0u, 0u);
  }
  lds_barrier();
  uint4 qb[16];  // B operand of k-step t: head l16, the dims of this lane group's chunk for t
  {
    const uint16_t* qrow = qlds + l16 * kQQRow;
#pragma unroll
    for (int t = 0; t < 14; ++t)
      qb[t] = *reinterpret_cast<const uint4*>(qrow + 16 * (grp + 4 * (t >> 1)) + 8 * (t & 1));
#pragma unroll
    for (int t = 14; t < 16; ++t) qb[t] = *reinterpret_cast<const uint4*>(qrow + kNope + 8 * (grp + 4 * (t - 14)));
  }
  if constexpr (Lay::ALIAS) lds_barrier();  // the query staging is overwritten by the V tiles below

  float x[SUBS][4];
#pragma unroll
  for (int j = 0; j < SUBS; ++j) {
    const int u = wave + NW * j;  // global sub-tile (wave-uniform)
    if (u >= nsub) {
#pragma unroll
      for (int e = 0; e < 4; ++e) x[j][e] = -INFINITY;
      continue;
    }
    const QRows& w = rw[j];
    const uint32_t valid16 = static_cast<uint32_t>(__ballot(w.ok) & 0xffffull);
    const bool any255 = __ballot(w.ok && has_scale_255(w.sc)) != 0ull;
    uint16_t* trow = vtile + (u * kQSub + l16) * VROW;  // dim d (of this part) of this slot at trow + d - DW part
    f32x4_t sacc0 = f32x4_t{0.f, 0.f, 0.f, 0.f}, sacc1 = sacc0;
    // The 7 e4m3 chunks, with the hardware conversion or (rare: a scale byte
    // of 255 in the sub-tile) the software decode -- one branch around the
    // whole sequence, so the common path's code is contiguous.
    auto nope = [&](auto sw) {
#pragma unroll
      for (int i = 0; i < 7; ++i) {
        const uint32_t sbyte = (i < 4 ? w.sc.x >> (8 * i) : w.sc.y >> (8 * (i - 4))) & 0xffu;
        uint4 lo, hi;
        if constexpr (decltype(sw)::value) {
          lo = dequant8_bf16_sw(make_uint2(w.c[i].x, w.c[i].y), sbyte);
          hi = dequant8_bf16_sw(make_uint2(w.c[i].z, w.c[i].w), sbyte);
        } else {
          lo = dequant8_bf16_hw(make_uint2(w.c[i].x, w.c[i].y), sbyte);
          hi = dequant8_bf16_hw(make_uint2(w.c[i].z, w.c[i].w), sbyte);
        }
        const int d = 16 * (grp + 4 * i);  // nope dims d .. d + 15 (a skipped slot's row is zero)
        if (d >= DW * part && d < DW * (part + 1)) {
          *reinterpret_cast<uint4*>(trow + (d - DW * part)) = lo;
          *reinterpret_cast<uint4*>(trow + (d - DW * part) + 8) = hi;
        }
        sacc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, lo),
                                                        __builtin_bit_cast(bf16x8_t, qb[2 * i]), sacc0, 0, 0, 0);
        sacc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, hi),
                                                        __builtin_bit_cast(bf16x8_t, qb[2 * i + 1]), sacc1, 0, 0, 0);
      }
    };
    if (!any255)
      nope(std::false_type{});
    else
      nope(std::true_type{});
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 rope = w.c[7 + i];
      const int d = kNope + 8 * (grp + 4 * i);  // rope dims d .. d + 7
      if (d >= DW * part && d < DW * (part + 1)) *reinterpret_cast<uint4*>(trow + (d - DW * part)) = rope;
      if (i == 0)
        sacc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, rope),
                                                        __builtin_bit_cast(bf16x8_t, qb[14]), sacc0, 0, 0, 0);
      else
        sacc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, rope),
                                                        __builtin_bit_cast(bf16x8_t, qb[15]), sacc1, 0, 0, 0);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      x[j][e] = ((valid16 >> (4 * grp + e)) & 1u) ? (sacc0[e] + sacc1[e]) * a.qscale : -INFINITY;
  }

  // ---- 3. softmax over the whole slot list ----------------------------------
  float mw = -INFINITY;
#pragma unroll
  for (int j = 0; j < SUBS; ++j)
#pragma unroll
    for (int e = 0; e < 4; ++e) mw = fmaxf(mw, x[j][e]);
  mw = fmaxf(mw, __uint_as_float(lane_xor<16>(__float_as_uint(mw), lane)));
  mw = fmaxf(mw, __uint_as_float(lane_xor<32>(__float_as_uint(mw), lane)));
  if (grp == 0) mxs[wave * 16 + l16] = mw;
  lds_barrier();  // maxima, and every V tile
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < NW; ++w) M = fmaxf(M, mxs[w * 16 + l16]);
  float ps = 0.f;
#pragma unroll
  for (int j = 0; j < SUBS; ++j) {
    float p[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      p[e] = M == -INFINITY ? 0.f : fast_exp2(x[j][e] - M);
      ps += p[e];
    }
    const int u = wave + NW * j;
    if (u < nsub)
      *reinterpret_cast<uint2*>(pt + l16 * kOpProw + u * kQSub + 4 * grp) =
          make_uint2(bf16x2_nb(p[0], p[1]), bf16x2_nb(p[2], p[3]));
  }
  ps += __uint_as_float(lane_xor<16>(__float_as_uint(ps), lane));
  ps += __uint_as_float(lane_xor<32>(__float_as_uint(ps), lane));
  if (grp == 0) lss[wave * 16 + l16] = ps;
  lds_barrier();  // P^T rows and sums

  // ---- 4. O^T = V^T P^T over every sub-tile, then the sink -----------------
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w) L += lss[w * 16 + l16];
  f32x4_t o[OB];
#pragma unroll
  for (int j = 0; j < OB; ++j) o[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // V^T A operand of output block b (dims 16 b .. of this part) of sub-tile
  // u: lane a of group g passes &V[16 u + 4 g + a / 4][16 b + 4 (a % 4)].
  // This wavefront's blocks are wave, wave + NW, ... (< NB; wave-uniform).
  const uint16_t* vbase = vtile + (4 * grp + l16 / 4) * VROW + 4 * (l16 % 4) + 16 * wave;
  const uint16_t* pbase = pt + l16 * kOpProw + 4 * grp;
  if (OB == 1 && wave < NB) {
    // One block per wavefront (four dim parts): sub-tile by sub-tile (the
    // grouped reads below measured ~0.1 us slower at nq 1 H 8).
    for (int u = 0; u < nsub; ++u) {
      const i16x4_t pb = __builtin_bit_cast(i16x4_t, *reinterpret_cast<const uint2*>(pbase + u * kQSub));
      const i16x4_t vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vbase + u * kQSub * VROW));
      o[0] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt, pb, o[0], 0, 0, 0);
    }
  } else if (wave < NB) {
    // The reads of kPvGroup sub-tiles are issued together, then their MFMAs
    // in sub-tile order (the chain of each block is unchanged), so one wait
    // covers a group instead of every sub-tile.  Nothing is under a branch:
    // a sub-tile past the list re-reads the last one with its probabilities
    // zeroed (its MFMA adds exact zeros: the V values are finite, and an
    // accumulator that starts at +0 never holds -0), and a block past NB
    // re-reads the last block (its sums are never stored).
    constexpr int kPvGroup = 4;
    for (int u0 = 0; u0 < nsub; u0 += kPvGroup) {
      i16x4_t pb[kPvGroup], vt[kPvGroup][OB];
#pragma unroll
      for (int i = 0; i < kPvGroup; ++i) {
        const int u = min(u0 + i, nsub - 1);
        const uint2 pw = *reinterpret_cast<const uint2*>(pbase + u * kQSub);
        pb[i] = __builtin_bit_cast(i16x4_t, u0 + i < nsub ? pw : make_uint2(0u, 0u));
#pragma unroll
        for (int j = 0; j < OB; ++j) {
          const int jb = min(wave + NW * j, NB - 1) - wave;
          vt[i][j] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vbase + u * kQSub * VROW + 16 * jb));
        }
      }
#pragma unroll
      for (int i = 0; i < kPvGroup; ++i)
#pragma unroll
        for (int j = 0; j < OB; ++j) o[j] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt[i][j], pb[i], o[j], 0, 0, 0);
    }
  }
  const float sk = g.sink ? sink_raw * kLog2e : -INFINITY;
  const float mx = L > 0.f ? fmaxf(sk, M) : sk;
  const float wgt = (L > 0.f && mx != -INFINITY) ? fast_exp2(M - mx) : 0.f;
  float Lt = wgt * (L > 0.f ? L : 0.f);
  if (g.sink && mx != -INFINITY) Lt += fast_exp2(sk - mx);
  const float sc = L != L ? __builtin_nanf("") : (Lt > 0.f ? wgt / Lt : 0.f);
  if (l16 < nh) {
    bf16* orow = g.out + (query * a.heads + h0 + l16) * kDim + DW * part + 16 * wave + 4 * grp;
#pragma unroll
    for (int j = 0; j < OB; ++j)
      if (wave + NW * j < NB)
        *reinterpret_cast<uint2*>(orow + 16 * NW * j) =
            make_uint2(bf16x2_nb(o[j][0] * sc, o[j][1] * sc), bf16x2_nb(o[j][2] * sc, o[j][3] * sc));
  }
}

constexpr int kMergeThreads = kDim / 4;  // 4 output columns per thread
constexpr int kMergeChunk = 1024;        // tile weights staged in LDS per pass
constexpr int kMergeFastTiles = 16;      // tiles merged straight from registers

// Merge of the tile partials with the sink as a virtual token of logit
// sink[h] and value 0 (csrc/dsv4_attention.cu:252-269): M = max(sink, m_t),
// L = 2^(sink-M) + sum_{l_t>0} l_t 2^(m_t-M), out = sum_t w_t acc_t / L with
// w_t = 2^(m_t-M) (0 for empty tiles).  Up to kMergeFastTiles tiles merge
// from registers in one round trip; beyond that the weights are computed in
// parallel into LDS and the column sums stream the partial rows.
template <typename T>
__global__ __launch_bounds__(kMergeThreads) void dsv4_merge_kernel(const float* __restrict__ part_ml,
                                                                   const float* __restrict__ part_acc,
                                                                   const float* __restrict__ sink,
                                                                   T* __restrict__ out, int heads,
                                                                   int num_tiles) {
  __shared__ float s_w[kMergeChunk];
  __shared__ float s_mx, s_inv;
  const int64_t qh = blockIdx.x;
  const int head = static_cast<int>(blockIdx.x % static_cast<uint32_t>(heads));  // 32-bit (grid < 2^32)
  const int tid = threadIdx.x;
  const float2* ml = reinterpret_cast<const float2*>(part_ml) + qh * num_tiles;
  if (num_tiles <= kMergeFastTiles) {
    // Few tiles: every (m, l) pair and every partial value this thread needs
    // is requested before the first wait (clamped tile indices, no branch
    // around a load), and each thread forms the weights itself -- one memory
    // round trip and no barrier.
    const int d = 4 * tid;
    const float* pa = part_acc + qh * num_tiles * static_cast<int64_t>(kDim) + d;
    float4 x[kMergeFastTiles];
    float2 v[kMergeFastTiles];
#pragma unroll
    for (int t = 0; t < kMergeFastTiles; ++t) {
      const int tt = t < num_tiles ? t : 0;
      x[t] = *reinterpret_cast<const float4*>(pa + static_cast<int64_t>(tt) * kDim);
      v[t] = ml[tt];
    }
    const float sk = sink ? sink[head] * kLog2e : -INFINITY;
    float mx = sk;
    bool nan_in = false;  // a NaN/inf score makes the softmax NaN, as torch.softmax does
#pragma unroll
    for (int t = 0; t < kMergeFastTiles; ++t) {
      if (t < num_tiles && v[t].y > 0.f) mx = fmaxf(mx, v[t].x);
      nan_in = nan_in || (t < num_tiles && v[t].y != v[t].y);
    }
    float L = 0.f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    if (mx != -INFINITY) {
#pragma unroll
      for (int t = 0; t < kMergeFastTiles; ++t) {
        if (t < num_tiles && v[t].y > 0.f) {
          const float w = fast_exp2(v[t].x - mx);
          L = fmaf(v[t].y, w, L);
          acc.x = fmaf(w, x[t].x, acc.x);
          acc.y = fmaf(w, x[t].y, acc.y);
          acc.z = fmaf(w, x[t].z, acc.z);
          acc.w = fmaf(w, x[t].w, acc.w);
        }
      }
      if (sink) L += fast_exp2(sk - mx);
    }
    const float inv = nan_in ? __builtin_nanf("") : (L > 0.f ? 1.f / L : 0.f);
    T* o = out + qh * kDim + d;
    o[0] = from_f32<T>(acc.x * inv);
    o[1] = from_f32<T>(acc.y * inv);
    o[2] = from_f32<T>(acc.z * inv);
    o[3] = from_f32<T>(acc.w * inv);
    return;
  }
  if (tid < kWave) {
    const float sk = sink ? sink[head] * kLog2e : -INFINITY;
    float mx = -INFINITY;
    bool nan_in = false;
    for (int t = tid; t < num_tiles; t += kWave) {
      const float2 v = ml[t];
      if (v.y > 0.f) mx = fmaxf(mx, v.x);
      nan_in = nan_in || v.y != v.y;
    }
    nan_in = __any(nan_in);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, xor_lanes(mx, off));
    mx = fmaxf(mx, sk);
    float L = 0.f;
    if (mx != -INFINITY) {
      for (int t = tid; t < num_tiles; t += kWave) {
        const float2 v = ml[t];
        if (v.y > 0.f) L += v.y * fast_exp2(v.x - mx);
      }
    }
    L = wave_sum(L);
    if (tid == 0) {
      if (sink && mx != -INFINITY) L += fast_exp2(sk - mx);
      s_mx = mx;
      s_inv = nan_in ? __builtin_nanf("") : (L > 0.f ? 1.f / L : 0.f);
    }
  }
  __syncthreads();
  const float mx = s_mx, inv = s_inv;
  const int d = 4 * tid;
  const float* pa = part_acc + qh * num_tiles * static_cast<int64_t>(kDim) + d;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int c0 = 0; c0 < num_tiles; c0 += kMergeChunk) {
    const int cn = min(kMergeChunk, num_tiles - c0);
    for (int t = tid; t < cn; t += kMergeThreads) {
      const float2 v = ml[c0 + t];
      s_w[t] = (v.y > 0.f && mx != -INFINITY) ? fast_exp2(v.x - mx) : 0.f;
    }
    __syncthreads();
#pragma unroll 8
    for (int t = 0; t < cn; ++t) {
      const float w = s_w[t];
      const float4 x = *reinterpret_cast<const float4*>(pa + static_cast<int64_t>(c0 + t) * kDim);
      acc.x = fmaf(w, x.x, acc.x);
      acc.y = fmaf(w, x.y, acc.y);
      acc.z = fmaf(w, x.z, acc.z);
      acc.w = fmaf(w, x.w, acc.w);
    }
    __syncthreads();
  }
  T* o = out + qh * kDim + d;
  o[0] = from_f32<T>(acc.x * inv);
  o[1] = from_f32<T>(acc.y * inv);
  o[2] = from_f32<T>(acc.z * inv);
  o[3] = from_f32<T>(acc.w * inv);
}

// Split selection: tile_size > 0 -> ceil(total/tile) tiles (csrc/dsv4_attention.cu:858-860);
// automatic -> about 2048 wavefronts over the device, at least 4 slots each.
void dsv4_tiling(int64_t nq, int64_t heads, int64_t total_slots, int64_t tile_size,
                 int64_t* tile_out, int64_t* tiles_out) {
  const int64_t total = std::max<int64_t>(1, total_slots);
  int64_t tiles;
  if (tile_size > 0) {
    tiles = ceil_div(total, tile_size);
  } else {
    const int64_t work = std::max<int64_t>(1, nq * ceil_div(std::max<int64_t>(1, heads), kHeadGroup));
    const int64_t want = std::max<int64_t>(1, ceil_div(2048, work));
    const int64_t max_tiles = std::max<int64_t>(1, ceil_div(total, 4));
    tiles = std::min(want, max_tiles);
  }
  const int64_t tile = ceil_div(total, tiles);
  *tile_out = tile;
  *tiles_out = ceil_div(total, tile);
}

size_t ws_bytes(int64_t nq, int64_t heads, int64_t tiles) {
  const size_t ml = static_cast<size_t>(nq * heads * tiles * 2) * sizeof(float);
  return ((ml + 255) & ~size_t{255}) + static_cast<size_t>(nq * heads * tiles * kDim) * sizeof(float);
}

// Workgroup target of the MFMA split (CSAHCA_DSV4_MFMA_WGS, read per call).
int64_t mfma_target_wgs() {
  const char* e = std::getenv("CSAHCA_DSV4_MFMA_WGS");
  const long v = e ? std::strtol(e, nullptr, 10) : 0;
  return v > 0 ? v : 256;
}

// MFMA path split of each query's slot list: enough (query, head group,
// split) workgroups for ~256 CUs, whole 32-slot tiles per split.
void mfma_splits(int64_t nq, int64_t heads, int64_t total_slots, int64_t* splits_out, int64_t* tps_out) {
  const int64_t groups = ceil_div(std::max<int64_t>(1, heads), kMfmaHeads);
  const int64_t ntiles = std::max<int64_t>(1, ceil_div(total_slots, kMfmaSlots));
  const int64_t wgs = std::max<int64_t>(1, nq * groups);
  const int64_t target = mfma_target_wgs();
  int64_t splits = wgs < target ? std::min(ntiles, ceil_div(target, wgs)) : 1;
  const int64_t tps = ceil_div(ntiles, splits);
  *splits_out = ceil_div(ntiles, tps);
  *tps_out = tps;
}

// CSAHCA_DSV4_MFMA=0 keeps every call on the VALU kernels (read per call).
bool mfma_enabled() {
  const char* e = std::getenv("CSAHCA_DSV4_MFMA");
  return !(e && e[0] == '0');
}

// The per-query kernel takes a call when there are at least 64 (query, head
// group) workgroups (measured per call, nq 32 x H 64: 13.5-13.6 us with two
// workgroups per (query, 16 heads) against 18.3-21.4 for the split kernel and
// its merge), or when the slot list is one round of 8 sub-tiles but more than
// one split tile (33-128 slots: no merge launch; the 128-slot window at nq 1
// and at nq 32 x H 8: 8.7-9.1 us against 8.8-9.8).  Longer lists at fewer
// workgroups stay on the split kernel (12 sub-tiles at nq 1: 12.1-12.7 us
// per-query against 8.8-9.5 split).
// CSAHCA_DSV4_QUERY=0 / =1 forces the choice (read per call).
bool use_query_kernel(int64_t nq, int64_t heads, int64_t total_slots) {
  const char* e = std::getenv("CSAHCA_DSV4_QUERY");
  if (e && (e[0] == '0' || e[0] == '1')) return e[0] == '1';
  const int64_t groups = ceil_div(std::max<int64_t>(1, heads), kQHeads);
  return nq * groups >= 64 || (total_slots > kMfmaSlots && total_slots <= 8 * kQSub);
}

// Wavefronts per workgroup of the per-query kernel (4 or 8; a round covers
// that many 16-slot sub-tiles): 8 where the slot list fits one round of 8
// (measured per launch, per-query kernel at nq 1-32 x H 8-64: the 128-slot
// SWA window 7-11% faster than two rounds of 4), else 4 (192 slots: two
// rounds of 8, the second half empty, are no faster than three of 4).
// CSAHCA_DSV4_QWAVES=4/8 forces either.
int query_waves(int64_t total_slots) {
  const char* e = std::getenv("CSAHCA_DSV4_QWAVES");
  if (e && (e[0] == '4' || e[0] == '8') && e[1] == 0) return e[0] - '0';
  return total_slots <= 8 * kQSub ? 8 : 4;
}

// Workgroups per (query, 16 heads) of the per-query kernel, each writing its
// share of the output dims: the most of 4, 2 and 1 at which the workgroups
// still fit one per CU.  CSAHCA_DSV4_QPARTS=1/2/4 forces a count.
int query_dim_parts(int64_t nq, int64_t groups) {
  const char* e = std::getenv("CSAHCA_DSV4_QPARTS");
  if (e && (e[0] == '1' || e[0] == '2' || e[0] == '4') && e[1] == 0) return e[0] - '0';
  const int ncu = device_cu_count();
  const int64_t base = ceil_div(nq, 8) * 8 * groups;
  if (ncu <= 0) return 1;
  return 4 * base <= ncu ? 4 : 2 * base <= ncu ? 2 : 1;
}

// The one-pass kernel takes every bf16 call with automatic tiling whose slot
// list fits it (1 .. kOpMaxSlots slots).  CSAHCA_DSV4_ONEPASS=0 turns it off,
// and so does CSAHCA_DSV4_QUERY=0 / 1, which forces the split / per-query
// kernel (both read per call).
bool use_onepass(int64_t total_slots) {
  const char* e = std::getenv("CSAHCA_DSV4_ONEPASS");
  if (e && e[0] == '0' && e[1] == 0) return false;
  const char* f = std::getenv("CSAHCA_DSV4_QUERY");
  if (f && (f[0] == '0' || f[0] == '1')) return false;
  return total_slots > 0 && total_slots <= kOpMaxSlots;
}

// Dim parts of the one-pass kernel: 4 where the workgroups still fit one per
// CU, else 2 (a part of all 512 dims would not fit the V tiles in LDS).
// CSAHCA_DSV4_QPARTS=2/4 forces a count.
int onepass_dim_parts(int64_t nq, int64_t groups) {
  const char* e = std::getenv("CSAHCA_DSV4_QPARTS");
  if (e && (e[0] == '2' || e[0] == '4') && e[1] == 0) return e[0] - '0';
  const int ncu = device_cu_count();
  const int64_t base = ceil_div(nq, 8) * 8 * groups;
  return (ncu > 0 && 4 * base <= ncu) ? 4 : 2;
}

struct Dsv4Call {
  const void* q;
  int dtype;
  int64_t nq, heads;
  CacheView swa, extra;
  const int32_t* idx;
  int64_t topk_slots;
  const int32_t* lens;
  const int32_t* eidx;
  int64_t extra_slots;
  const int32_t* elens;
  const float* sink;
  double softmax_scale;
  int64_t tile_size;
  void* out;
  void* workspace;
  size_t workspace_bytes;
  void* stream;
};

int dsv4_run(const Dsv4Call& c) {
  if (c.nq == 0 || c.heads == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(c.q && c.out, "null tensor pointer");
  CSAHCA_REQUIRE(c.idx || c.topk_slots == 0 || c.nq == 0, "null token_indices pointer");
  const int64_t total = c.topk_slots + c.extra_slots;
  CSAHCA_REQUIRE(total <= INT_MAX && c.nq <= INT_MAX && c.heads <= INT_MAX, "too many slots");
  const bool vec = reinterpret_cast<uintptr_t>(c.swa.base) % 16 == 0 && c.swa.bpp % 16 == 0 &&
                   (c.extra_slots == 0 ||
                    (reinterpret_cast<uintptr_t>(c.extra.base) % 16 == 0 && c.extra.bpp % 16 == 0));
  // Grouped-head MFMA path: bf16 queries, automatic split, 16-byte aligned rows.
  const bool use_mfma = c.dtype == CSAHCA_BF16 && c.tile_size == 0 && vec &&
                        reinterpret_cast<uintptr_t>(c.q) % 16 == 0 && mfma_enabled();
  int64_t tile, tiles, tps = 0;
  if (use_mfma) {
    mfma_splits(c.nq, c.heads, total, &tiles, &tps);
    tile = tps * kMfmaSlots;
  } else {
    dsv4_tiling(c.nq, c.heads, total, c.tile_size, &tile, &tiles);
  }
  const int64_t head_groups = ceil_div(c.heads, kHeadGroup);
  CSAHCA_REQUIRE(c.nq * head_groups * tiles <= INT32_MAX, "too many DSV4 work items");
  const size_t need = ws_bytes(c.nq, c.heads, tiles);
  if (c.workspace == nullptr || c.workspace_bytes < need)
    return fail(CSAHCA_ERR_WORKSPACE, "workspace too small for dsv4 decode");
  Dsv4Args a;
  a.swa = c.swa;
  a.extra = c.extra;
  a.idx = c.idx;
  a.lens = c.lens;
  a.eidx = c.eidx;
  a.elens = c.elens;
  a.part_ml = static_cast<float*>(c.workspace);
  const size_t ml = static_cast<size_t>(c.nq * c.heads * tiles * 2) * sizeof(float);
  a.part_acc = reinterpret_cast<float*>(static_cast<char*>(c.workspace) + ((ml + 255) & ~size_t{255}));
  a.heads = static_cast<int>(c.heads);
  a.head_groups = static_cast<int>(head_groups);
  a.topk_slots = static_cast<int>(c.topk_slots);
  a.extra_slots = static_cast<int>(c.extra_slots);
  a.tile = static_cast<int>(tile);
  a.num_tiles = static_cast<int>(tiles);
  a.qscale = static_cast<float>(c.softmax_scale) * kLog2e;
  hipStream_t stream = static_cast<hipStream_t>(c.stream);
  if (use_mfma && reinterpret_cast<uintptr_t>(c.out) % 8 == 0 && use_onepass(total)) {
    QueryArgs qa;
    qa.nq = c.nq;
    qa.groups = static_cast<int>(ceil_div(c.heads, kQHeads));
    qa.nsub = static_cast<int>(ceil_div(total, kQSub));
    qa.sink = c.sink;
    qa.out = static_cast<bf16*>(c.out);
    const int ds = onepass_dim_parts(c.nq, qa.groups);
    // query q's (group, part) pairs x: blocks q%8 + 8 (x + G DS q/8)
    const int64_t blocks = ceil_div(c.nq, 8) * 8 * qa.groups * ds;
    CSAHCA_REQUIRE(blocks <= INT32_MAX, "too many DSV4 work items");
    // 12 wavefronts with one sub-tile each for lists of up to 192 slots, else
    // 8 with two (CSAHCA_DSV4_OPWAVES=8 / 12 forces either where it fits).
    const char* ew = std::getenv("CSAHCA_DSV4_OPWAVES");
    const bool w12 = ew ? (std::atoi(ew) == 12 && total <= 12 * kQSub) : total <= 12 * kQSub;
    auto kfn = w12 ? (ds == 4 ? dsv4_onepass_kernel<12, 1, 4> : dsv4_onepass_kernel<12, 1, 2>)
                   : (ds == 4 ? dsv4_onepass_kernel<8, 2, 4> : dsv4_onepass_kernel<8, 2, 2>);
    return launch("dsv4_onepass_kernel", kfn, dim3(static_cast<uint32_t>(blocks)), dim3((w12 ? 12 : 8) * kWave),
                  0, stream, a.idx, a.eidx, a.lens, a.elens, a.topk_slots, a.extra_slots, qa.groups,
                  static_cast<int32_t>(qa.nq), a.heads, static_cast<const bf16*>(c.q), a, qa);
  }
  if (use_mfma && reinterpret_cast<uintptr_t>(c.out) % 8 == 0 && use_query_kernel(c.nq, c.heads, total)) {
    QueryArgs qa;
    qa.nq = c.nq;
    qa.groups = static_cast<int>(ceil_div(c.heads, kQHeads));
    qa.nsub = static_cast<int>(ceil_div(total, kQSub));
    qa.sink = c.sink;
    qa.out = static_cast<bf16*>(c.out);
    const int ds = query_dim_parts(c.nq, qa.groups);
    // query q's (group, part) pairs x: blocks q%8 + 8 (x + G DS q/8)
    const int64_t blocks = ceil_div(c.nq, 8) * 8 * qa.groups * ds;
    CSAHCA_REQUIRE(blocks <= INT32_MAX, "too many DSV4 work items");
    const bool w8 = query_waves(total) == 8;
    auto kfn = w8 ? (ds == 4 ? dsv4_query_kernel<8, 4> : ds == 2 ? dsv4_query_kernel<8, 2> : dsv4_query_kernel<8, 1>)
                  : (ds == 4 ? dsv4_query_kernel<4, 4> : ds == 2 ? dsv4_query_kernel<4, 2> : dsv4_query_kernel<4, 1>);
    return launch("dsv4_query_kernel", kfn, dim3(static_cast<uint32_t>(blocks)), dim3((w8 ? 8 : 4) * kWave), 0,
                  stream, static_cast<const bf16*>(c.q), a, qa);
  }
  if (use_mfma) {
    MfmaArgs mm;
    mm.splits = static_cast<int>(tiles);
    mm.tiles_per_split = static_cast<int>(tps);
    mm.mfma_groups = static_cast<int>(ceil_div(c.heads, kMfmaHeads));
    mm.sink = c.sink;
    mm.out = static_cast<bf16*>(c.out);
    const dim3 mgrid(static_cast<uint32_t>(c.nq * mm.mfma_groups * tiles));
    const bf16* qp = static_cast<const bf16*>(c.q);
    // One split (a slot list of at most one 32-slot tile per workgroup): the
    // workgroup merges with the sink itself, no merge launch.
    if (tiles == 1)
      return launch("dsv4_mfma_kernel", dsv4_mfma_kernel<kMfmaDirect>, mgrid, dim3(kMfmaThreads), 0, stream, qp, a,
                    mm);
    const int rc = launch("dsv4_mfma_kernel", dsv4_mfma_kernel<kMfmaPartials>, mgrid, dim3(kMfmaThreads), 0, stream,
                          qp, a, mm);
    if (rc != CSAHCA_OK) return rc;
    return launch("dsv4_merge_kernel", dsv4_merge_kernel<bf16>, dim3(static_cast<uint32_t>(c.nq * c.heads)),
                  dim3(kMergeThreads), 0, stream, static_cast<const float*>(a.part_ml),
                  static_cast<const float*>(a.part_acc), c.sink, static_cast<bf16*>(c.out), a.heads, a.num_tiles);
  }
  const dim3 grid(static_cast<uint32_t>(c.nq * head_groups * tiles));
  return dispatch_dtype(c.dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    const T* qp = static_cast<const T*>(c.q);
    const bool tvec = vec && reinterpret_cast<uintptr_t>(c.q) % 16 == 0;
    const int rc = tvec ? launch("dsv4_tile_kernel", dsv4_tile_kernel<T, true>, grid, dim3(kWave), 0,
                                stream, qp, a)
                       : launch("dsv4_tile_kernel", dsv4_tile_kernel<T, false>, grid, dim3(kWave), 0,
                                stream, qp, a);
    if (rc != CSAHCA_OK) return rc;
    return launch("dsv4_merge_kernel", dsv4_merge_kernel<T>,
                  dim3(static_cast<uint32_t>(c.nq * c.heads)), dim3(kMergeThreads), 0, stream,
                  static_cast<const float*>(a.part_ml), static_cast<const float*>(a.part_acc), c.sink,
                  static_cast<T*>(c.out), a.heads, a.num_tiles);
  });
}

int check_common(int dtype, int64_t nq, int64_t heads, int64_t bpp, int64_t page_size,
                 int64_t num_pages, int64_t topk_slots) {
  CSAHCA_REQUIRE(valid_dtype(dtype), "q must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(nq >= 0 && heads >= 0 && topk_slots >= 0 && num_pages >= 0 && bpp >= 0,
                 "negative dimension");
  CSAHCA_REQUIRE(page_size > 0, "page_size must be positive");
  CSAHCA_REQUIRE(page_size <= INT_MAX, "page_size must fit in int32");
  CSAHCA_REQUIRE(bpp >= page_size * (kRowBytes + kScaleBytes),
                 "bytes_per_page is too small for DSV4 page layout");
  return CSAHCA_OK;
}

}  // namespace
}  // namespace csahca

using namespace csahca;

extern "C" size_t csahca_dsv4_decode_workspace_bytes(int64_t num_queries, int64_t heads,
                                                     int64_t topk_slots, int64_t extra_topk_slots,
                                                     int64_t tile_size) {
  if (num_queries < 0 || heads < 0 || topk_slots < 0 || extra_topk_slots < 0) return 0;
  int64_t tile, tiles, splits, tps;
  dsv4_tiling(num_queries, heads, topk_slots + extra_topk_slots, tile_size, &tile, &tiles);
  mfma_splits(num_queries, heads, topk_slots + extra_topk_slots, &splits, &tps);
  // either path may run (the MFMA one for bf16 queries with automatic tiling)
  return ws_bytes(num_queries, heads, tile_size > 0 ? tiles : std::max(tiles, splits));
}

extern "C" int csahca_dsv4_decode_forward_tiled(
    const void* q, int dtype, int64_t num_queries, int64_t heads, const uint8_t* cache,
    int64_t num_pages, int64_t bytes_per_page, int64_t page_size, const int32_t* token_indices,
    int64_t topk_slots, const int32_t* topk_lengths, const uint8_t* extra_cache,
    int64_t extra_num_pages, int64_t extra_bytes_per_page, int64_t extra_page_size,
    const int32_t* extra_token_indices, int64_t extra_topk_slots,
    const int32_t* extra_topk_lengths, const float* attn_sink, double softmax_scale,
    int64_t tile_size, void* out, void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_common(dtype, num_queries, heads, bytes_per_page, page_size, num_pages, topk_slots);
  if (rc != CSAHCA_OK) return rc;
  CSAHCA_REQUIRE(bytes_per_page % 4 == 0,
                 "tiled DSV4 kernel requires bytes_per_page divisible by 4 for vectorized loads");
  CSAHCA_REQUIRE(tile_size >= 0, "tile_size must be non-negative");
  const bool has_extra = extra_cache != nullptr && extra_num_pages * extra_bytes_per_page > 0 &&
                         extra_token_indices != nullptr && num_queries * extra_topk_slots > 0;
  Dsv4Call c{};
  if (has_extra) {
    CSAHCA_REQUIRE(extra_page_size > 0, "extra_page_size must be positive");
    CSAHCA_REQUIRE(extra_page_size <= INT_MAX, "extra_page_size must fit in int32");
    CSAHCA_REQUIRE(extra_bytes_per_page >= extra_page_size * (kRowBytes + kScaleBytes),
                   "extra_bytes_per_page is too small for DSV4 page layout");
    CSAHCA_REQUIRE(extra_bytes_per_page % 4 == 0,
                   "tiled DSV4 kernel requires extra_bytes_per_page divisible by 4 for vectorized loads");
    c.extra = cache_view(extra_cache, extra_num_pages, extra_bytes_per_page, extra_page_size);
    c.eidx = extra_token_indices;
    c.extra_slots = extra_topk_slots;
    c.elens = extra_topk_lengths;
  }
  c.q = q;
  c.dtype = dtype;
  c.nq = num_queries;
  c.heads = heads;
  c.swa = cache_view(cache, num_pages, bytes_per_page, page_size);
  c.idx = token_indices;
  c.topk_slots = topk_slots;
  c.lens = topk_lengths;
  c.sink = attn_sink;
  c.softmax_scale = softmax_scale;
  c.tile_size = tile_size;
  c.out = out;
  c.workspace = workspace;
  c.workspace_bytes = workspace_bytes;
  c.stream = stream;
  return dsv4_run(c);
}

extern "C" int csahca_dsv4_swa_decode_forward(const void* q, int dtype, int64_t num_queries,
                                              int64_t heads, const uint8_t* cache,
                                              int64_t num_pages, int64_t bytes_per_page,
                                              int64_t page_size, const int32_t* token_indices,
                                              int64_t topk_slots, const int32_t* topk_lengths,
                                              const float* attn_sink, double softmax_scale,
                                              void* out, void* workspace, size_t workspace_bytes,
                                              void* stream) {
  clear_error();
  int rc = check_common(dtype, num_queries, heads, bytes_per_page, page_size, num_pages, topk_slots);
  if (rc != CSAHCA_OK) return rc;
  Dsv4Call c{};
  c.q = q;
  c.dtype = dtype;
  c.nq = num_queries;
  c.heads = heads;
  c.swa = cache_view(cache, num_pages, bytes_per_page, page_size);
  c.idx = token_indices;
  c.topk_slots = topk_slots;
  c.lens = topk_lengths;
  c.sink = attn_sink;
  c.softmax_scale = softmax_scale;
  c.tile_size = 0;
  c.out = out;
  c.workspace = workspace;
  c.workspace_bytes = workspace_bytes;
  c.stream = stream;
  return dsv4_run(c);
}

extern "C" int csahca_dsv4_sparse_decode_forward(
    const void* q, int dtype, int64_t num_queries, int64_t heads, const uint8_t* cache,
    int64_t num_pages, int64_t bytes_per_page, int64_t page_size, const int32_t* token_indices,
    int64_t topk_slots, const int32_t* topk_lengths, const uint8_t* extra_cache,
    int64_t extra_num_pages, int64_t extra_bytes_per_page, int64_t extra_page_size,
    const int32_t* extra_token_indices, int64_t extra_topk_slots,
    const int32_t* extra_topk_lengths, const float* attn_sink, double softmax_scale, void* out,
    void* workspace, size_t workspace_bytes, void* stream) {
  clear_error();
  int rc = check_common(dtype, num_queries, heads, bytes_per_page, page_size, num_pages, topk_slots);
  if (rc != CSAHCA_OK) return rc;
  CSAHCA_REQUIRE(extra_page_size > 0, "extra_page_size must be positive");
  CSAHCA_REQUIRE(extra_page_size <= INT_MAX, "extra_page_size must fit in int32");
  CSAHCA_REQUIRE(extra_num_pages >= 0 && extra_topk_slots >= 0, "negative dimension");
  CSAHCA_REQUIRE(extra_bytes_per_page >= extra_page_size * (kRowBytes + kScaleBytes),
                 "extra_bytes_per_page is too small for DSV4 page layout");
  Dsv4Call c{};
  const bool has_extra = extra_cache != nullptr && extra_token_indices != nullptr &&
                         extra_topk_slots > 0;
  if (has_extra) {
    c.extra = cache_view(extra_cache, extra_num_pages, extra_bytes_per_page, extra_page_size);
    c.eidx = extra_token_indices;
    c.extra_slots = extra_topk_slots;
    c.elens = extra_topk_lengths;
  }
  c.q = q;
  c.dtype = dtype;
  c.nq = num_queries;
  c.heads = heads;
  c.swa = cache_view(cache, num_pages, bytes_per_page, page_size);
  c.idx = token_indices;
  c.topk_slots = topk_slots;
  c.lens = topk_lengths;
  c.sink = attn_sink;
  c.softmax_scale = softmax_scale;
  c.tile_size = 0;
  c.out = out;
  c.workspace = workspace;
  c.workspace_bytes = workspace_bytes;
  c.stream = stream;
  return dsv4_run(c);
}
