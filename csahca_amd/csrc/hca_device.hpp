// hca_device.hpp -- the HCA chunk pass as a device function: one 256-thread
// workgroup pools one chunk of K and V (fp32 column sums, means rounded to the
// storage type), scores the K mean against q and writes (score, V mean).  Used
// by the HCA kernel and by the hybrid kernel, which runs it beside the CSA step.
#pragma once
#include "common.hpp"

namespace csahca {

constexpr int kHcaThreads = 256;

// Rows of K and V in flight per thread (4: 128 B of loads per lane.  Measured
// chunk pass, chunk 256, D 128: B1 H8 S32768 level with 8 at 0.68-0.69 of 8
// TB/s; B4 0.71 against 0.68 for 8 and 0.64 for 16 -- more bytes in flight per
// lane than the memory system drains only queue.)
constexpr int kRowBatch = 4;

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
__device__ __forceinline__ void hca_chunk_body(const T* __restrict__ q, const T* __restrict__ k,
                                               const T* __restrict__ v, float* __restrict__ scores,
                                               float* __restrict__ means, int64_t S, int D, int chunk,
                                               int64_t C, float scale, int64_t item) {
  constexpr int VEC = kVec ? Vec16<T>::N : 1;
  extern __shared__ float lds[];
  __shared__ float red[kHcaThreads / kWave];
  const int tid = threadIdx.x;
  // 32-bit division whenever the item index fits (every practical shape).
  int64_t bh, c;
  if (item <= static_cast<int64_t>(UINT32_MAX) && C <= static_cast<int64_t>(UINT32_MAX)) {
    const uint32_t it = static_cast<uint32_t>(item), cc = static_cast<uint32_t>(C);
    const uint32_t b32 = it / cc;
    bh = b32;
    c = it - b32 * cc;
  } else {
    bh = item / C;
    c = item - bh * C;
  }
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

}  // namespace csahca
