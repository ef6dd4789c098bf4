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
//                     means, scores the K mean against q and writes the
//                     score (scores[b,h,c]) and the V mean (means[b,h,c,:])
//                     to the workspace;
//   hca_merge_kernel  one workgroup per (b, h, block of 32 output columns):
//                     softmax over the C scores, probabilities rounded to the
//                     storage type, sum of its columns of the V means,
//                     optional blend with a CSA output.  Spreading a head's
//                     columns over workgroups keeps each one to a single round
//                     trip of ~C x 128 bytes even at batch 1.
#include "common.hpp"

#include <algorithm>
#include <climits>
#include <cmath>

namespace csahca {
namespace {

constexpr int kHcaThreads = 256;
constexpr int kHcaProbChunk = 2048;  // probabilities staged in LDS per pass

constexpr int kRowBatch = 8;          // rows of K and V in flight per thread

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
                                                              float* __restrict__ scores,
                                                              float* __restrict__ means, int64_t S,
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
      // The loads are unconditional (rows past the chunk re-read row r0 and
      // are zeroed after the load): a load under a per-lane branch would make
      // the compiler wait for the whole batch before issuing it.
      for (int r0 = rg; r0 < chunk; r0 += kRowBatch * R) {
        if constexpr (kVec) {
          uint4 rk[kRowBatch], rv[kRowBatch];
#pragma unroll
          for (int i = 0; i < kRowBatch; ++i) {
            const int r = r0 + i * R;
            const int64_t off = static_cast<int64_t>(r < chunk ? r : r0) * D;
            rk[i] = load_global_u4(kc + off);
            rv[i] = load_global_u4(vcp + off);
          }
          // Keep the scheduler from interleaving the widening below with the
          // loads (it would wait for the first rows before requesting the rest).
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int i = 0; i < kRowBatch; ++i) {
            const bool ok = r0 + i * R < chunk;
            float xk[VEC], xv[VEC];
            widen16<T>(rk[i], xk);
            widen16<T>(rv[i], xv);
#pragma unroll
            for (int e = 0; e < VEC; ++e) {
              ak[e] += ok ? xk[e] : 0.f;
              av[e] += ok ? xv[e] : 0.f;
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
  float* out = means + item * static_cast<int64_t>(D);
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
    out[d] = vm;
  }
  dot = block_reduce(dot, red, false);
  if (tid == 0) scores[item] = dot * scale;
}

// Merge thread layout: 32 columns x 8 row groups; a wavefront reads 2 rows of
// 128 contiguous bytes per load.  When C <= 256 every score and every V-mean
// value a thread needs is requested before the first wait (one round trip);
// larger C runs in passes of kHcaProbChunk rows, kMergeRows rows per batch.
constexpr int kMergeCols = 32;
constexpr int kMergeRowGroups = kHcaThreads / kMergeCols;  // 8
constexpr int kMergeRows = 32;                             // rows per thread per batch
constexpr int kMergeFastRows = kMergeRows * kMergeRowGroups;  // 256
static_assert(kMergeFastRows <= kHcaThreads, "one score per thread in the one-round-trip path");

template <typename T>
__global__ __launch_bounds__(kHcaThreads) void hca_merge_kernel(const float* __restrict__ scores,
                                                              const float* __restrict__ means,
                                                              const T* __restrict__ blend,
                                                              float w_csa, T* __restrict__ out,
                                                              int64_t C, int D, int col_blocks) {
  __shared__ float s_p[kHcaProbChunk];
  __shared__ float s_sum[kHcaThreads];
  __shared__ float red[kHcaThreads / kWave];
  const int tid = threadIdx.x;
  const int64_t bh = blockIdx.x / col_blocks;
  const int cb = static_cast<int>(blockIdx.x - bh * col_blocks);
  const int rg = tid / kMergeCols, cl = tid % kMergeCols;
  const int d = cb * kMergeCols + cl;
  const bool has_col = d < D;
  const float* sb = scores + bh * C;
  const float* col = means + bh * C * D + (has_col ? d : 0);  // column 0 stands in: loads stay in bounds

  float a = 0.f;
  if (C <= kMergeFastRows) {
    const int n = static_cast<int>(C);
    // Unconditional loads (clamped indices, values dropped after the load):
    // the score and the V-mean column values are one batch in flight.
    const float sraw = load_global_raw<float>(sb + (tid < n ? tid : 0));
    float x[kMergeRows];
#pragma unroll
    for (int i = 0; i < kMergeRows; ++i) {
      const int r = rg + i * kMergeRowGroups;
      x[i] = load_global_raw<float>(col + static_cast<int64_t>(r < n ? r : 0) * D);
    }
    const float sc = tid < n ? sraw : -INFINITY;
    const float M = block_reduce(sc, red, true);
    const float e = (tid < n && M != -INFINITY) ? fast_exp2((sc - M) * kLog2e) : 0.f;
    const float L = block_reduce(e, red, false);
    const float iv = L > 0.f ? 1.f / L : 0.f;
    // softmax in fp32, then the cast of the probabilities to the V dtype
    if (tid < n) s_p[tid] = round_to<T>(e * iv);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kMergeRows; ++i) {
      const int r = rg + i * kMergeRowGroups;
      if (r < n) a = fmaf(s_p[r], x[i], a);
    }
  } else {
    float mx = -INFINITY;
    for (int64_t c = tid; c < C; c += kHcaThreads) mx = fmaxf(mx, sb[c]);
    mx = block_reduce(mx, red, true);
    float L = 0.f;
    if (mx != -INFINITY)
      for (int64_t c = tid; c < C; c += kHcaThreads) L += fast_exp2((sb[c] - mx) * kLog2e);
    L = block_reduce(L, red, false);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    for (int64_t p0 = 0; p0 < C; p0 += kHcaProbChunk) {
      const int pn = static_cast<int>(std::min<int64_t>(kHcaProbChunk, C - p0));
      for (int c = tid; c < pn; c += kHcaThreads)
        s_p[c] = mx != -INFINITY ? round_to<T>(fast_exp2((sb[p0 + c] - mx) * kLog2e) * inv) : 0.f;
      __syncthreads();
      const float* cp = col + p0 * D;
      for (int r0 = rg; r0 < pn; r0 += kMergeRows * kMergeRowGroups) {
        float x[kMergeRows];
#pragma unroll
        for (int i = 0; i < kMergeRows; ++i) {
          const int r = r0 + i * kMergeRowGroups;
          x[i] = cp[static_cast<int64_t>(r < pn ? r : r0) * D];
        }
#pragma unroll
        for (int i = 0; i < kMergeRows; ++i) {
          const int r = r0 + i * kMergeRowGroups;
          if (r < pn) a = fmaf(s_p[r], x[i], a);
        }
      }
      __syncthreads();
    }
  }
  s_sum[tid] = a;
  __syncthreads();
  if (rg == 0 && has_col) {
    float o = 0.f;
#pragma unroll
    for (int g = 0; g < kMergeRowGroups; ++g) o += s_sum[g * kMergeCols + cl];
    o = round_to<T>(o);
    if (blend) {
      // w*csa + (1-w)*hca with each product and the sum rounded to T
      const float ab = round_to<T>(w_csa * to_f32(blend[bh * D + d]));
      const float bb = round_to<T>((1.f - w_csa) * o);
      o = ab + bb;
    }
    out[bh * D + d] = from_f32<T>(o);
  }
}

}  // namespace
}  // namespace csahca

using namespace csahca;

namespace {
// Workspace: scores f32[B*H*C], then (256-byte aligned) means f32[B*H*C*D].
size_t hca_means_offset(int64_t n_scores) {
  return (static_cast<size_t>(n_scores) * sizeof(float) + 255) & ~size_t{255};
}
}  // namespace

extern "C" size_t csahca_hca_decode_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len,
                                                   int64_t head_dim, int64_t chunk_size) {
  if (batch < 0 || heads < 0 || seq_len < 0 || head_dim < 0 || chunk_size <= 0) return 0;
  const int64_t C = seq_len / chunk_size;
  return hca_means_offset(batch * heads * C) + static_cast<size_t>(batch * heads * C * head_dim) * sizeof(float);
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
  float* scores = static_cast<float*>(workspace);
  float* means = reinterpret_cast<float*>(static_cast<char*>(workspace) + hca_means_offset(bh * C));
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
                     kp, vp, scores, means, seq_len, D, static_cast<int>(chunk_size), C, scale)
            : launch("hca_chunk_kernel", hca_chunk_kernel<T, false>, grid, dim3(kHcaThreads), lds, stream, qp,
                     kp, vp, scores, means, seq_len, D, static_cast<int>(chunk_size), C, scale);
    if (rc != CSAHCA_OK) return rc;
    const int col_blocks = (D + kMergeCols - 1) / kMergeCols;
    CSAHCA_REQUIRE(bh * col_blocks <= INT32_MAX, "too many heads in one call");
    return launch("hca_merge_kernel", hca_merge_kernel<T>, dim3(static_cast<uint32_t>(bh * col_blocks)),
                  dim3(kHcaThreads), 0, stream, static_cast<const float*>(scores),
                  static_cast<const float*>(means), static_cast<const T*>(blend_src),
                  static_cast<float>(blend_weight), static_cast<T*>(out), C, D, col_blocks);
  });
}
