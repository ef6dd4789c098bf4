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
#include "hca_device.hpp"

#include <algorithm>
#include <climits>
#include <cmath>

namespace csahca {
namespace {

constexpr int kHcaProbChunk = 2048;  // probabilities staged in LDS per pass

// Parameter order: the inputs of the first loads (q, K, V and the sizes that
// place them) lead, so they fit the 14 dwords preloaded into SGPRs at wave
// launch (the library builds this file with -amdgpu-kernarg-preload-count);
// the outputs and the scale, needed at the end, follow.
template <typename T, bool kVec>
__global__ __launch_bounds__(kHcaThreads) void hca_chunk_kernel(const T* __restrict__ q,
                                                              const T* __restrict__ k,
                                                              const T* __restrict__ v, int64_t S,
                                                              int64_t C, int D, int chunk,
                                                              float* __restrict__ scores,
                                                              float* __restrict__ means, float scale) {
  hca_chunk_body<T, kVec>(q, k, v, scores, means, S, D, chunk, C, scale, blockIdx.x);
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
                     kp, vp, seq_len, C, D, static_cast<int>(chunk_size), scores, means, scale)
            : launch("hca_chunk_kernel", hca_chunk_kernel<T, false>, grid, dim3(kHcaThreads), lds, stream, qp,
                     kp, vp, seq_len, C, D, static_cast<int>(chunk_size), scores, means, scale);
    if (rc != CSAHCA_OK) return rc;
    const int col_blocks = (D + kMergeCols - 1) / kMergeCols;
    CSAHCA_REQUIRE(bh * col_blocks <= INT32_MAX, "too many heads in one call");
    return launch("hca_merge_kernel", hca_merge_kernel<T>, dim3(static_cast<uint32_t>(bh * col_blocks)),
                  dim3(kHcaThreads), 0, stream, static_cast<const float*>(scores),
                  static_cast<const float*>(means), static_cast<const T*>(blend_src),
                  static_cast<float>(blend_weight), static_cast<T*>(out), C, D, col_blocks);
  });
}

namespace csahca {

// The HCA merge (+ optional blend) from a workspace a chunk pass of shape
// (bh, C, D) filled; used by the hybrid step, which runs the chunk pass inside
// its own kernel.
int hca_merge_launch(int dtype, void* workspace, const void* blend_src, double blend_weight, void* out,
                     int64_t bh, int64_t C, int D, hipStream_t stream) {
  const float* scores = static_cast<const float*>(workspace);
  const float* means =
      reinterpret_cast<const float*>(static_cast<const char*>(workspace) + hca_means_offset(bh * C));
  const int col_blocks = (D + kMergeCols - 1) / kMergeCols;
  CSAHCA_REQUIRE(bh * col_blocks <= INT32_MAX, "too many heads in one call");
  return dispatch_dtype(dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    return launch("hca_merge_kernel", hca_merge_kernel<T>, dim3(static_cast<uint32_t>(bh * col_blocks)),
                  dim3(kHcaThreads), 0, stream, scores, means, static_cast<const T*>(blend_src),
                  static_cast<float>(blend_weight), static_cast<T*>(out), C, D, col_blocks);
  });
}

// Byte offset of the V means in an HCA workspace holding n chunk scores.
size_t hca_workspace_means_offset(int64_t n_scores) { return hca_means_offset(n_scores); }

}  // namespace csahca
