// block.hip -- the matrix-vector products of a decode block, for gfx950.
//
// A decode step multiplies a few token rows (batch <= 4) by weight matrices
// in torch's nn.Linear layout W[out_features, in_features].  At this size the
// product is a stream over W (2 bytes per weight, 2 flops per weight and
// token row): HBM-bound, so it runs on the VALU with 16-byte loads, not on
// MFMA.  One kernel covers every product of the hybrid decode block, with
// the neighbouring elementwise work fused in:
//   prologue  optional RMSNorm of the input rows,
//             x * rsqrt(mean(x^2) + eps) * g rounded to the storage type;
//   epilogue  the product rounded to the storage type, then either
//             an optional activation (SiLU or exact GELU), an optional
//             + residual and an optional base + alpha * (.), each rounded;
//             or the QKV scatter: q to [B,H,D], k and v appended to
//             [B,H,capacity,D] caches at the device-side position, and the
//             count of complete chunks after that token;
//             optionally the device position advanced by one.
// Rounding points follow the torch ops they replace (F.linear output, F.silu /
// F.gelu of the rounded product, the bf16 residual add, `hidden + 0.01 * out`).
//
// Work split: a wavefront owns kRowsPerWave rows of W; lane l owns the
// 16-byte column chunks l, l + 64, ... of a row, so a row of K values is
// K/512 loads per lane and a workgroup of 4 wavefronts reads 4 kRowsPerWave
// rows.  Every load of a wavefront -- input rows, norm weights, weight rows,
// residuals, the position -- is issued unconditionally as one batch (clamped
// indices, values dropped after the loads), so the kernel is one HBM round
// trip plus the reduction.
#include "common.hpp"

#include <climits>

namespace csahca {
namespace {

constexpr int kGemvWaves = 4;
constexpr int kGemvThreads = kGemvWaves * kWave;
constexpr int kRowsPerWave = 2;

enum GemvEpilogue : int { kEpiGeneral = 0, kEpiQkv = 1 };

struct GemvArgs {
  const void* x;      // [B, K]
  const void* norm;   // [K] RMSNorm weight, or null
  float eps;
  const void* w;      // [N, K]
  int act;            // CSAHCA_ACT_*
  const void* res;    // [B, N] residual, or null
  const void* base;   // [B, N] base of base + alpha * y, or null
  float alpha;
  void* y;            // [B, N] (kEpiGeneral)
  // kEpiQkv: N = 3 H D; output n = (part, head, dim) in that order
  void* q;            // [B, H, D]
  void* kc;           // [B, H, capacity, D]
  void* vc;
  const int64_t* pos; // token position written
  int32_t* nchunks;   // complete chunks after the token, or null
  int64_t capacity;
  int heads, head_dim, chunk;
  int64_t* advance;   // position advanced by one at the end, or null
  int B, N, K;
};

template <typename T>
__device__ __forceinline__ float round_t(float v) {
  return to_f32(from_f32<T>(v));
}

template <typename T, int KV, int BB, int EPI>
// The leading scalars repeat the arguments of the kernel's one batch of loads
// (x, the weights, the norm weight, the residual and base rows, the sizes);
// the library preloads them into SGPRs at wave launch, so the weight stream
// is requested without waiting for an argument load.  The copies in `a` are
// the same values.
__global__ __launch_bounds__(kGemvThreads) void block_gemv_kernel(const void* x_, const void* w_, const void* norm,
                                                                  const void* res, const void* base, int32_t B,
                                                                  int32_t N, int32_t K, GemvArgs a) {
  a.x = x_;
  a.w = w_;
  a.norm = norm;
  a.res = res;
  a.base = base;
  a.B = B;
  a.N = N;
  a.K = K;
  constexpr int RW = kRowsPerWave;
  constexpr int NV = BB * RW;  // outputs of a wavefront
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const int n0 = (static_cast<int>(blockIdx.x) * kGemvWaves + wave) * RW;
  const int kc = a.K / 8;  // 16-byte chunks per row
  const T* __restrict__ x = static_cast<const T*>(a.x);
  const T* __restrict__ w = static_cast<const T*>(a.w);
  const bool has_norm = a.norm != nullptr;

  // ---- one batch of loads ------------------------------------------------
  uint4 xr[BB][KV], gr[KV], wr[RW][KV];
#pragma unroll
  for (int j = 0; j < KV; ++j) {
    const int c = lane + kWave * j;
    const int cc = c < kc ? c : 0;
#pragma unroll
    for (int b = 0; b < BB; ++b)
      xr[b][j] = load_global_u4(x + static_cast<int64_t>(b < a.B ? b : 0) * a.K + 8 * cc);
    gr[j] = load_global_u4(has_norm ? static_cast<const void*>(static_cast<const T*>(a.norm) + 8 * cc)
                                    : static_cast<const void*>(x + 8 * cc));
  }
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = n0 + r < a.N ? n0 + r : a.N - 1;
#pragma unroll
    for (int j = 0; j < KV; ++j) {
      const int c = lane + kWave * j;
      wr[r][j] = load_global_u4(w + static_cast<int64_t>(n) * a.K + 8 * (c < kc ? c : 0));
    }
  }
  // The output this lane stores (lanes < NV): batch row ob, weight row n0 + orow.
  const int oi = lane < NV ? lane : 0;
  const int ob = oi / RW, orow = oi % RW;
  const int on = n0 + orow;
  const bool store = lane < NV && ob < a.B && on < a.N;
  float resv = 0.f, basev = 0.f;
  if constexpr (EPI == kEpiGeneral) {
    // (absent operands re-read x[0] and are dropped)
    const int64_t ri = static_cast<int64_t>(ob < a.B ? ob : 0) * a.N + (on < a.N ? on : a.N - 1);
    resv = to_f32(load_global_elem<T>(a.res ? static_cast<const T*>(a.res) + ri : x));
    basev = to_f32(load_global_elem<T>(a.base ? static_cast<const T*>(a.base) + ri : x));
  }
  int64_t pos = 0;
  if constexpr (EPI == kEpiQkv) pos = load_global_raw<int64_t>(a.pos);
  __builtin_amdgcn_sched_barrier(0);

  // ---- prologue: widen (and normalise) the input rows --------------------
  float xf[BB][KV][8];
#pragma unroll
  for (int b = 0; b < BB; ++b)
#pragma unroll
    for (int j = 0; j < KV; ++j) {
      widen16<T>(xr[b][j], xf[b][j]);
      const bool live = lane + kWave * j < kc;
#pragma unroll
      for (int e = 0; e < 8; ++e) xf[b][j][e] = live ? xf[b][j][e] : 0.f;
    }
  if (has_norm) {
    float g[KV][8];
#pragma unroll
    for (int j = 0; j < KV; ++j) widen16<T>(gr[j], g[j]);
    float ss[BB];
#pragma unroll
    for (int b = 0; b < BB; ++b) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < KV; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) s = fmaf(xf[b][j][e], xf[b][j][e], s);
      ss[b] = s;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
      for (int b = 0; b < BB; ++b) ss[b] += xor_lanes(ss[b], off);
#pragma unroll
    for (int b = 0; b < BB; ++b) {
      const float rs = rsqrtf(ss[b] / static_cast<float>(a.K) + a.eps);
#pragma unroll
      for (int j = 0; j < KV; ++j)
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[b][j][e] = round_t<T>(xf[b][j][e] * rs * g[j][e]);
    }
  }

  // ---- products and their wavefront sums ---------------------------------
  float acc[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) acc[i] = 0.f;
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int j = 0; j < KV; ++j) {
      float wf[8];
      widen16<T>(wr[r][j], wf);
#pragma unroll
      for (int b = 0; b < BB; ++b)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[b * RW + r] = fmaf(xf[b][j][e], wf[e], acc[b * RW + r]);
    }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
    for (int i = 0; i < NV; ++i) acc[i] += xor_lanes(acc[i], off);
  float v = acc[0];
#pragma unroll
  for (int i = 1; i < NV; ++i) v = lane == i ? acc[i] : v;

  // ---- epilogue ----------------------------------------------------------
  const float y0 = round_t<T>(v);
  if constexpr (EPI == kEpiQkv) {
    if (store) {
      const int hd = a.heads * a.head_dim;
      const int part = on / hd, rem = on - part * hd;
      const int h = rem / a.head_dim, d = rem - h * a.head_dim;
      const int64_t bh = static_cast<int64_t>(ob) * a.heads + h;
      if (part == 0)
        static_cast<T*>(a.q)[bh * a.head_dim + d] = from_f32<T>(y0);
      else if (pos >= 0 && pos < a.capacity)  // a position outside the cache writes no K/V
        static_cast<T*>(part == 1 ? a.kc : a.vc)[(bh * a.capacity + pos) * a.head_dim + d] = from_f32<T>(y0);
    }
    if (a.nchunks != nullptr && blockIdx.x == 0 && threadIdx.x == 0)
      *a.nchunks = static_cast<int32_t>((pos + 1) / a.chunk);
  } else {
    float out = y0;
    if (a.act == CSAHCA_ACT_SILU) out = round_t<T>(out / (1.f + __expf(-out)));
    if (a.act == CSAHCA_ACT_GELU) out = round_t<T>(0.5f * out * (1.f + erff(out * 0.70710678118654752f)));
    if (a.res != nullptr) out = round_t<T>(out + resv);
    if (a.base != nullptr) out = round_t<T>(basev + round_t<T>(a.alpha * out));
    if (store) static_cast<T*>(a.y)[static_cast<int64_t>(ob) * a.N + on] = from_f32<T>(out);
  }
  if (a.advance != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *a.advance = *a.advance + 1;
}

template <typename T, int KV, int BB>
int launch_gemv_epi(int epi, const GemvArgs& a, dim3 grid, hipStream_t stream) {
  const dim3 block(kGemvThreads);
  return epi == kEpiQkv
             ? launch("block_gemv_kernel", block_gemv_kernel<T, KV, BB, kEpiQkv>, grid, block, 0, stream, a.x, a.w,
                      a.norm, a.res, a.base, a.B, a.N, a.K, a)
             : launch("block_gemv_kernel", block_gemv_kernel<T, KV, BB, kEpiGeneral>, grid, block, 0, stream, a.x,
                      a.w, a.norm, a.res, a.base, a.B, a.N, a.K, a);
}

template <typename T, int KV>
int launch_gemv_kv(int epi, const GemvArgs& a, dim3 grid, hipStream_t stream) {
  if constexpr (KV > 4) {
    return launch_gemv_epi<T, KV, 1>(epi, a, grid, stream);  // batch 1 only (checked on the host)
  } else {
    return a.B == 1 ? launch_gemv_epi<T, KV, 1>(epi, a, grid, stream) : launch_gemv_epi<T, KV, 4>(epi, a, grid, stream);
  }
}

template <typename T>
int launch_gemv(int epi, const GemvArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<uint32_t>(ceil_div(a.N, kGemvWaves * kRowsPerWave)));
  const int kv = static_cast<int>(ceil_div(a.K / 8, kWave));
  if (kv <= 1) return launch_gemv_kv<T, 1>(epi, a, grid, stream);
  if (kv <= 2) return launch_gemv_kv<T, 2>(epi, a, grid, stream);
  if (kv <= 4) return launch_gemv_kv<T, 4>(epi, a, grid, stream);
  return launch_gemv_kv<T, 8>(epi, a, grid, stream);
}

int check_gemv(int dtype, int64_t batch, int64_t n, int64_t k) {
  CSAHCA_REQUIRE(dtype == CSAHCA_BF16 || dtype == CSAHCA_F16, "decode block products support bfloat16 and float16");
  CSAHCA_REQUIRE(batch >= 0 && n >= 0 && k >= 0, "negative dimension");
  CSAHCA_REQUIRE(batch <= 4, "decode block products take at most 4 token rows");
  CSAHCA_REQUIRE(k % 8 == 0 && k <= 4096, "in_features must be a multiple of 8 and at most 4096");
  CSAHCA_REQUIRE(batch <= 1 || k <= 2048, "in_features above 2048 needs batch 1");
  CSAHCA_REQUIRE(n <= INT_MAX / 2, "out_features too large");
  return CSAHCA_OK;
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int run_gemv(int dtype, int epi, const GemvArgs& a, hipStream_t stream) {
  return dtype == CSAHCA_BF16 ? launch_gemv<bf16>(epi, a, stream) : launch_gemv<f16>(epi, a, stream);
}

}  // namespace
}  // namespace csahca

using namespace csahca;

extern "C" int csahca_block_linear(const void* x, const void* norm_weight, double eps, const void* weight,
                                   int activation, const void* residual, const void* base, double alpha,
                                   void* y, int dtype, int64_t batch, int64_t out_features,
                                   int64_t in_features, int64_t* advance_pos, void* stream) {
  clear_error();
  int rc = check_gemv(dtype, batch, out_features, in_features);
  if (rc != CSAHCA_OK) return rc;
  CSAHCA_REQUIRE(activation == CSAHCA_ACT_NONE || activation == CSAHCA_ACT_SILU || activation == CSAHCA_ACT_GELU,
                 "unknown activation");
  if ((batch == 0 || out_features == 0) && advance_pos == nullptr) return CSAHCA_OK;
  CSAHCA_REQUIRE(in_features > 0, "in_features must be positive");
  CSAHCA_REQUIRE(batch > 0 && out_features > 0, "advancing the position needs a non-empty product");
  CSAHCA_REQUIRE(x && weight && y, "null tensor pointer");
  CSAHCA_REQUIRE(aligned16(x) && aligned16(weight) && (!norm_weight || aligned16(norm_weight)),
                 "x, weight and norm_weight must be 16-byte aligned");
  GemvArgs a{};
  a.x = x;
  a.norm = norm_weight;
  a.eps = static_cast<float>(eps);
  a.w = weight;
  a.act = activation;
  a.res = residual;
  a.base = base;
  a.alpha = static_cast<float>(alpha);
  a.y = y;
  a.advance = advance_pos;
  a.B = static_cast<int>(batch);
  a.N = static_cast<int>(out_features);
  a.K = static_cast<int>(in_features);
  return run_gemv(dtype, kEpiGeneral, a, static_cast<hipStream_t>(stream));
}

extern "C" int csahca_block_qkv(const void* hidden, const void* norm_weight, double eps, const void* w_qkv,
                                void* q, void* k_cache, void* v_cache, const int64_t* token_pos,
                                int32_t* num_chunks, int dtype, int64_t batch, int64_t heads, int64_t head_dim,
                                int64_t capacity, int64_t chunk_size, void* stream) {
  clear_error();
  CSAHCA_REQUIRE(heads >= 0 && head_dim >= 0 && capacity >= 0, "negative dimension");
  const int64_t hidden_dim = heads * head_dim;
  int rc = check_gemv(dtype, batch, 3 * hidden_dim, hidden_dim);
  if (rc != CSAHCA_OK) return rc;
  CSAHCA_REQUIRE(chunk_size > 0 && chunk_size <= INT_MAX, "chunk_size must be positive");
  if (batch == 0 || hidden_dim == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(hidden && w_qkv && q && k_cache && v_cache, "null tensor pointer");
  CSAHCA_REQUIRE(token_pos, "null token_pos pointer");
  CSAHCA_REQUIRE(aligned16(hidden) && aligned16(w_qkv) && (!norm_weight || aligned16(norm_weight)),
                 "hidden, w_qkv and norm_weight must be 16-byte aligned");
  GemvArgs a{};
  a.x = hidden;
  a.norm = norm_weight;
  a.eps = static_cast<float>(eps);
  a.w = w_qkv;
  a.q = q;
  a.kc = k_cache;
  a.vc = v_cache;
  a.pos = token_pos;
  a.nchunks = num_chunks;
  a.capacity = capacity;
  a.heads = static_cast<int>(heads);
  a.head_dim = static_cast<int>(head_dim);
  a.chunk = static_cast<int>(chunk_size);
  a.B = static_cast<int>(batch);
  a.N = static_cast<int>(3 * hidden_dim);
  a.K = static_cast<int>(hidden_dim);
  return run_gemv(dtype, kEpiQkv, a, static_cast<hipStream_t>(stream));
}
