// hca.hip -- heavily compressed attention (HCA) decode and the CSA/HCA hybrid
// blend, for gfx950.
//
// hca_reference (hybrid_attention/reference.py:87-92): K and V are mean-pooled
// per chunk (fp32 mean, then rounded to the storage type) and the query
// attends to all C = S/chunk summary rows with full softmax attention whose
// probabilities are rounded to the storage type before the PV product
// (reference.py:31-37).  hybrid_reference (reference.py:95-108) blends
// w*csa + (1-w)*hca with each product and the sum rounded to the storage type.
//
// Kernels:
//   hca_chunk_kernel  one workgroup per (b, h, chunk) streams the chunk's K and
//                     V rows with 16-byte lane loads (the whole op is one pass
//                     over K and V: HBM-bound), reduces them to the two rounded
//                     means, scores the K mean against q and writes
//                     (score, V mean) to the workspace;
//   hca_merge_kernel  one workgroup per (b, h): softmax over the C scores,
//                     probabilities rounded to the storage type, sum of the V
//                     means, optional blend with a CSA output.
#include "common.hpp"

#include <algorithm>
#include <climits>
#include <cmath>

namespace csahca {
namespace {

constexpr int kHcaThreads = 256;
constexpr int kHcaProbChunk = 2048;  // probabilities staged in LDS per pass

constexpr int kRowBatch = 8;          // rows of K and V in flight per thread

// Widen one 16-byte load of T to fp32.
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

template <typename T>
__device__ __forceinline__ float round_to(float x) {
  return to_f32(from_f32<T>(x));
}

__device__ __forceinline__ float block_reduce(float v, float* red, bool is_max) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = xor_lanes(v, off);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < kHcaThreads / kWave; ++w) r = is_max ? fmaxf(r, red[w]) : r + red[w];
  return r;
}

// Thread layout over one chunk: tpr threads per row (each owning VEC-wide
// column groups, looping when a row has more than 256 groups), R = 256/tpr
// rows per pass.  LDS: 2 x R x D fp32 row-group sums, then the block reduce.
template <typename T, bool kVec>
__global__ __launch_bounds__(kHcaThreads) void hca_chunk_kernel(const T* __restrict__ q,
                                                              const T* __restrict__ k,
                                                              const T* __restrict__ v,
                                                              float* __restrict__ part, int64_t S,
                                                              int D, int chunk, int64_t C,
                                                              float scale) {
  constexpr int VEC = kVec ? Vec16<T>::N : 1;
  extern __shared__ float lds[];
  __shared__ float red[kHcaThreads / kWave];
  const int tid = threadIdx.x;
  const int64_t item = blockIdx.x;
  const int64_t bh = item / C;
  const int64_t c = item - bh * C;
  const int nvc = D / VEC;
  const int tpr = min(nvc, kHcaThreads);
  const int R = kHcaThreads / tpr;
  const int rg = tid / tpr;
  const int lc = tid - rg * tpr;
  float* sk = lds;
  float* sv = lds + static_cast<size_t>(R) * D;
  const int64_t row0 = bh * S + c * chunk;

  if (rg < R) {
    for (int vc = lc; vc < nvc; vc += tpr) {
      float ak[VEC], av[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) ak[e] = av[e] = 0.f;
      const T* kc = k + row0 * D + static_cast<int64_t>(vc) * VEC;
      const T* vcp = v + row0 * D + static_cast<int64_t>(vc) * VEC;
      // kRowBatch rows of K and V are requested before any is consumed, so a
      // thread waits for one HBM round trip per batch rather than per row.
      for (int r0 = rg; r0 < chunk; r0 += kRowBatch * R) {
        if constexpr (kVec) {
          uint4 rk[kRowBatch], rv[kRowBatch];
#pragma unroll
          for (int i = 0; i < kRowBatch; ++i) {
            const int r = r0 + i * R;
            const int64_t off = static_cast<int64_t>(r < chunk ? r : r0) * D;
            rk[i] = *reinterpret_cast<const uint4*>(kc + off);
            rv[i] = *reinterpret_cast<const uint4*>(vcp + off);
          }
#pragma unroll
          for (int i = 0; i < kRowBatch; ++i) {
            if (r0 + i * R < chunk) {
              float xk[VEC], xv[VEC];
              widen16<T>(rk[i], xk);
              widen16<T>(rv[i], xv);
#pragma unroll
              for (int e = 0; e < VEC; ++e) {
                ak[e] += xk[e];
                av[e] += xv[e];
              }
            }
          }
        } else {
          float xk[kRowBatch], xv[kRowBatch];
#pragma unroll
          for (int i = 0; i < kRowBatch; ++i) {
            const int r = r0 + i * R;
            const int64_t off = static_cast<int64_t>(r < chunk ? r : r0) * D;
            xk[i] = to_f32(kc[off]);
            xv[i] = to_f32(vcp[off]);
          }
#pragma unroll
          for (int i = 0; i < kRowBatch; ++i) {
            if (r0 + i * R < chunk) {
              ak[0] += xk[i];
              av[0] += xv[i];
            }
          }
        }
      }
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        sk[rg * D + vc * VEC + e] = ak[e];
        sv[rg * D + vc * VEC + e] = av[e];
      }
    }
  }
  __syncthreads();
  // Column means, rounded to the storage type; the score partial q . kmean.
  const float inv_n = 1.f / static_cast<float>(chunk);
  const T* qp = q + bh * D;
  float* out = part + item * (static_cast<int64_t>(D) + 1);
  float dot = 0.f;
  for (int d = tid; d < D; d += kHcaThreads) {
    float a = 0.f, b = 0.f;
    for (int g = 0; g < R; ++g) {
      a += sk[g * D + d];
      b += sv[g * D + d];
    }
    const float km = round_to<T>(a * inv_n);
    const float vm = round_to<T>(b * inv_n);
    dot = fmaf(to_f32(qp[d]), km, dot);
    out[1 + d] = vm;
  }
  dot = block_reduce(dot, red, false);
  if (tid == 0) out[0] = dot * scale;
}

// Thread layout of the PV sum: RG = 256/D row groups (1 when D > 256) x D
// columns; each thread keeps kMergeBatch rows of its column in flight, and the
// RG partial sums meet in LDS at the end.
constexpr int kMergeBatch = 64;         // rows per thread in the one-round-trip path
constexpr int kMergeBatchGeneral = 32;  // rows per thread per batch otherwise

template <typename T>
__global__ __launch_bounds__(kHcaThreads) void hca_merge_kernel(const float* __restrict__ part,
                                                              const T* __restrict__ blend,
                                                              float w_csa, T* __restrict__ out,
                                                              int64_t C, int D) {
  constexpr int kCols = 1024 / kHcaThreads;  // columns per thread when D > 256 (D <= 1024)
  __shared__ float s_p[kHcaProbChunk];
  __shared__ float s_sum[kHcaThreads];
  __shared__ float red[kHcaThreads / kWave];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.x;
  const int64_t stride = static_cast<int64_t>(D) + 1;
  const float* pb = part + bh * C * stride;
  const int RG = D <= kHcaThreads ? kHcaThreads / D : 1;
  const int tpc = D <= kHcaThreads ? D : kHcaThreads;  // threads per row group
  const int rg = tid / tpc;
  const int c0l = tid - rg * tpc;

  if (D <= kHcaThreads && C <= kHcaProbChunk && C <= static_cast<int64_t>(kMergeBatch) * RG) {
    // Common shape: every score and every V-mean value this thread needs is
    // requested before the first wait -- one memory round trip in total.
    constexpr int kScores = kHcaProbChunk / kHcaThreads;
    const int n = static_cast<int>(C);
    float sc[kScores], x[kMergeBatch];
#pragma unroll
    for (int j = 0; j < kScores; ++j) {
      const int c = tid + j * kHcaThreads;
      sc[j] = c < n ? pb[static_cast<int64_t>(c) * stride] : -INFINITY;
    }
    const bool mine = rg < RG;
    const float* col = pb + 1 + (mine ? c0l : 0);
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      const int r = rg + i * RG;
      x[i] = col[static_cast<int64_t>(mine && r < n ? r : 0) * stride];
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kScores; ++j) m = fmaxf(m, sc[j]);
    const float M = block_reduce(m, red, true);
    float l = 0.f;
    if (M != -INFINITY) {
#pragma unroll
      for (int j = 0; j < kScores; ++j)
        if (tid + j * kHcaThreads < n) l += fast_exp2((sc[j] - M) * kLog2e);
    }
    const float Lt = block_reduce(l, red, false);
    const float iv = Lt > 0.f ? 1.f / Lt : 0.f;
#pragma unroll
    for (int j = 0; j < kScores; ++j) {
      const int c = tid + j * kHcaThreads;
      // softmax in fp32, then the cast of the probabilities to the V dtype
      if (c < n) s_p[c] = M != -INFINITY ? round_to<T>(fast_exp2((sc[j] - M) * kLog2e) * iv) : 0.f;
    }
    __syncthreads();
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < kMergeBatch; ++i) {
      const int r = rg + i * RG;
      if (mine && r < n) a = fmaf(s_p[r], x[i], a);
    }
    s_sum[tid] = a;
    __syncthreads();
    if (tid < D) {
      float o = 0.f;
      for (int g = 0; g < RG; ++g) o += s_sum[g * D + tid];
      o = round_to<T>(o);
      if (blend) {
        // w*csa + (1-w)*hca with each product and the sum rounded to T
        const float ab = round_to<T>(w_csa * to_f32(blend[bh * D + tid]));
        const float bb = round_to<T>((1.f - w_csa) * o);
        o = ab + bb;
      }
      out[bh * D + tid] = from_f32<T>(o);
    }
    return;
  }

  float mx = -INFINITY;
  for (int64_t c = tid; c < C; c += kHcaThreads) mx = fmaxf(mx, pb[c * stride]);
  mx = block_reduce(mx, red, true);
  float L = 0.f;
  if (mx != -INFINITY)
    for (int64_t c = tid; c < C; c += kHcaThreads) L += fast_exp2((pb[c * stride] - mx) * kLog2e);
  L = block_reduce(L, red, false);
  const float inv = L > 0.f ? 1.f / L : 0.f;

  float acc[kCols];
#pragma unroll
  for (int j = 0; j < kCols; ++j) acc[j] = 0.f;
  for (int64_t p0 = 0; p0 < C; p0 += kHcaProbChunk) {
    const int pn = static_cast<int>(std::min<int64_t>(kHcaProbChunk, C - p0));
    for (int c = tid; c < pn; c += kHcaThreads) {
      const float x = pb[(p0 + c) * stride];
      // softmax in fp32, then the cast of the probabilities to the V dtype
      s_p[c] = mx != -INFINITY ? round_to<T>(fast_exp2((x - mx) * kLog2e) * inv) : 0.f;
    }
    __syncthreads();
    if (rg < RG) {
#pragma unroll
      for (int j = 0; j < kCols; ++j) {
        const int d = c0l + j * tpc;
        if (d < D) {
          const float* col = pb + p0 * stride + 1 + d;
          float a = acc[j];
          for (int r0 = rg; r0 < pn; r0 += kMergeBatchGeneral * RG) {
            float x[kMergeBatchGeneral];
#pragma unroll
            for (int i = 0; i < kMergeBatchGeneral; ++i) {
              const int r = r0 + i * RG;
              x[i] = col[static_cast<int64_t>(r < pn ? r : r0) * stride];
            }
#pragma unroll
            for (int i = 0; i < kMergeBatchGeneral; ++i) {
              const int r = r0 + i * RG;
              if (r < pn) a = fmaf(s_p[r], x[i], a);
            }
          }
          acc[j] = a;
        }
      }
    }
    __syncthreads();
  }
  // Sum the row groups (RG > 1 only when D <= 128: one column per thread).
  if (RG > 1) {
    s_sum[tid] = acc[0];
    __syncthreads();
    if (tid < D) {
      float a = 0.f;
      for (int g = 0; g < RG; ++g) a += s_sum[g * D + tid];
      acc[0] = a;
    }
  }
  if (rg == 0) {
#pragma unroll
    for (int j = 0; j < kCols; ++j) {
      const int d = c0l + j * tpc;
      if (d < D) {
        float o = round_to<T>(acc[j]);
        if (blend) {
          // w*csa + (1-w)*hca with each product and the sum rounded to T
          const float a = round_to<T>(w_csa * to_f32(blend[bh * D + d]));
          const float b = round_to<T>((1.f - w_csa) * o);
          o = a + b;
        }
        out[bh * D + d] = from_f32<T>(o);
      }
    }
  }
}

}  // namespace
}  // namespace csahca

using namespace csahca;

extern "C" size_t csahca_hca_decode_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len,
                                                   int64_t head_dim, int64_t chunk_size) {
  if (batch < 0 || heads < 0 || seq_len < 0 || head_dim < 0 || chunk_size <= 0) return 0;
  const int64_t C = seq_len / chunk_size;
  return static_cast<size_t>(batch * heads * C * (head_dim + 1)) * sizeof(float);
}

extern "C" int csahca_hca_decode_forward(const void* q, const void* k_cache, const void* v_cache,
                                         const void* blend_src, double blend_weight, void* out,
                                         int dtype, int64_t batch, int64_t heads, int64_t seq_len,
                                         int64_t head_dim, int64_t chunk_size, void* workspace,
                                         size_t workspace_bytes, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(valid_dtype(dtype), "q, k_cache and v_cache must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(batch >= 0 && heads >= 0 && seq_len >= 0 && head_dim >= 0, "negative dimension");
  CSAHCA_REQUIRE(chunk_size > 0 && chunk_size <= INT_MAX, "chunk_size must be positive");
  CSAHCA_REQUIRE(seq_len % chunk_size == 0, "seq length must be divisible by chunk_size");
  CSAHCA_REQUIRE(head_dim <= 1024, "head_dim > 1024 is not supported");
  const int64_t bh = batch * heads;
  if (bh == 0 || head_dim == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(q && k_cache && v_cache && out, "null tensor pointer");
  const int64_t C = seq_len / chunk_size;
  if (C == 0) return fail(CSAHCA_ERR_ARGUMENT, "seq length must be at least chunk_size");
  CSAHCA_REQUIRE(bh * C <= INT32_MAX, "too many chunks in one call");
  const size_t need = csahca_hca_decode_workspace_bytes(batch, heads, seq_len, head_dim, chunk_size);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CSAHCA_ERR_WORKSPACE, "workspace too small for hca decode");
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  float* part = static_cast<float*>(workspace);
  const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(head_dim)));
  const int D = static_cast<int>(head_dim);
  return dispatch_dtype(dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    constexpr int VEC = Vec16<T>::N;
    const bool vec = D % VEC == 0 &&
                     ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) % 16) == 0;
    const int nvc = vec ? D / VEC : D;
    const int R = kHcaThreads / std::min(nvc, kHcaThreads);
    const size_t lds = 2 * static_cast<size_t>(R) * D * sizeof(float);
    const dim3 grid(static_cast<uint32_t>(bh * C));
    const T* qp = static_cast<const T*>(q);
    const T* kp = static_cast<const T*>(k_cache);
    const T* vp = static_cast<const T*>(v_cache);
    const int rc =
        vec ? launch("hca_chunk_kernel", hca_chunk_kernel<T, true>, grid, dim3(kHcaThreads), lds, stream, qp,
                     kp, vp, part, seq_len, D, static_cast<int>(chunk_size), C, scale)
            : launch("hca_chunk_kernel", hca_chunk_kernel<T, false>, grid, dim3(kHcaThreads), lds, stream, qp,
                     kp, vp, part, seq_len, D, static_cast<int>(chunk_size), C, scale);
    if (rc != CSAHCA_OK) return rc;
    return launch("hca_merge_kernel", hca_merge_kernel<T>, dim3(static_cast<uint32_t>(bh)),
                  dim3(kHcaThreads), 0, stream, static_cast<const float*>(part),
                  static_cast<const T*>(blend_src), static_cast<float>(blend_weight), static_cast<T*>(out), C,
                  D);
  });
}
