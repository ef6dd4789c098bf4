// csa.hip -- CSA decode kernels for gfx950 and their C-ABI entry points.
//
// Decode step (one query token per (batch, head)):
//   1. csa_summary_*   : fp32 mean of every chunk of K (the chunk summaries).
//   2. csa_score_*     : score[c] = (q . summary[c]) / sqrt(D) in fp32, stored as
//                        an order-preserving uint32 key.
//   3. csa_topk_kernel : per (b,h) one wavefront loads the keys into LDS once and
//                        selects the top-k (radix select + rank; score desc,
//                        chunk id asc).
//   4. csa_attend_*    : split-KV sparse attention.  Work item = one wavefront
//                        over `tile` consecutive selected-token slots of one
//                        (b,h); K/V rows are fetched with 16-byte lane loads so
//                        one wavefront-wide load moves whole rows; online
//                        softmax in registers; fp32 partial (m, l, acc[D]).
//   5. csa_merge_kernel: log-sum-exp merge of the partials of each (b,h), with
//                        all partial loads independent of each other.
// csa_step.hip fuses 2-5 into one launch.  All offsets are 64-bit.
#include "csa_device.hpp"

#include <algorithm>
#include <climits>

namespace csahca {
namespace {

// ---------------------------------------------------------------------------
// Split-KV sparse attention (vectorised path).
// ---------------------------------------------------------------------------
// Parameter order: what the chunk-id load, the K/V row addresses and q need
// comes first (14 dwords, preloaded into SGPRs at wave launch: the library
// builds this file with -amdgpu-kernarg-preload-count), the outputs after;
// the chunk shift is formed here from the chunk size.
template <typename T, typename IdxT, int D, int U>
__global__ __launch_bounds__(64) void csa_attend_vec_kernel(
    const IdxT* __restrict__ idx, int64_t seq_len, const T* __restrict__ k, const T* __restrict__ v,
    const T* __restrict__ q, int num_tiles, int top_k, int tile, int chunk, float* __restrict__ part_ml,
    float* __restrict__ part_acc, float qscale) {
  const int chunk_shift = (chunk & (chunk - 1)) == 0 ? __builtin_ctz(static_cast<uint32_t>(chunk)) : -1;
  using L = AttendLayout<T, D>;
  constexpr int VEC = L::VEC, LPR = L::LPR, RPL = L::RPL;
  const int lane = threadIdx.x;
  const int grp = lane / LPR;
  const int col = lane % LPR;
  // 32-bit index arithmetic (the grid is < 2^32 blocks): a 64-bit division is
  // a long scalar sequence at the head of every workgroup.
  const uint32_t item = blockIdx.x;
  const int t = static_cast<int>(item % static_cast<uint32_t>(num_tiles));
  const int64_t bh = item / static_cast<uint32_t>(num_tiles);

  const T* qp = q + bh * D + col * VEC;
  const T* __restrict__ kb = k + bh * seq_len * D + col * VEC;
  const T* __restrict__ vb = v + bh * seq_len * D + col * VEC;
  const IdxT* __restrict__ ib = idx + bh * top_k;
  const int total = top_k * chunk;
  const int s0 = t * tile;
  const int s1 = min(s0 + tile, total);
  auto get_id = [&](int cs) { return ib[cs]; };
  auto tok_of = [&](int s, int64_t& tok) {
    return slot_token_of(get_id, s, chunk, chunk_shift, seq_len, tok);
  };
  WaveSoftmax<T, D> st;
  st.init();
  for (int base = s0; base < s1; base += RPL * U)
    attend_block<T, D, U>(st, qp, qscale, kb, vb, base, s1, grp, tok_of);
  // Row groups folded transposed: every lane stores kKeep of its columns' sums.
  const int fbase = fold_row_groups_share(st);
  const int64_t p = bh * num_tiles + t;
  {
    float* dst = part_acc + p * D + col * VEC + fbase;
#pragma unroll
    for (int e = 0; e < FoldShare<T, D>::kKeep; ++e) dst[e] = st.acc[e];
  }
  if (lane == 0) {
    part_ml[2 * p] = st.m;
    part_ml[2 * p + 1] = st.l;
  }
}

// Generic path: any D <= 64 * J, any storage type.  Lanes stride the columns
// (coalesced), kGenericRows rows per iteration, wavefront-wide dot reductions.
constexpr int kGenericRows = 4;
template <typename T, typename IdxT, int J>
__global__ __launch_bounds__(64) void csa_attend_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const IdxT* __restrict__ idx, float* __restrict__ part_ml, float* __restrict__ part_acc,
    int64_t seq_len, int D, int top_k, int chunk, int chunk_shift, int tile, int num_tiles,
    float qscale) {
  const int lane = threadIdx.x;
  // 32-bit index arithmetic (the grid is < 2^32 blocks): a 64-bit division is
  // a long scalar sequence at the head of every workgroup.
  const uint32_t item = blockIdx.x;
  const int t = static_cast<int>(item % static_cast<uint32_t>(num_tiles));
  const int64_t bh = item / static_cast<uint32_t>(num_tiles);
  float qf[J], acc[J];
  T qr[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int d = lane + kWave * j;
    qr[j] = load_global_elem<T>(q + bh * D + (d < D ? d : 0));  // one batch; columns past D dropped
  }
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int d = lane + kWave * j;
    qf[j] = d < D ? to_f32(qr[j]) * qscale : 0.f;
    acc[j] = 0.f;
  }
  const T* __restrict__ kb = k + bh * seq_len * D;
  const T* __restrict__ vb = v + bh * seq_len * D;
  const IdxT* __restrict__ ib = idx + bh * top_k;
  auto get_id = [&](int cs) { return ib[cs]; };
  const int total = top_k * chunk;
  const int s0 = t * tile;
  const int s1 = min(s0 + tile, total);
  float m = -INFINITY, l = 0.f;
  // kGenericRows slots per batch: their chunk ids, then their K and V rows,
  // are each requested unconditionally as one batch (slots past the tile
  // re-read its last slot, skipped slots and columns past D re-read row 0 /
  // column 0; all are dropped after the loads).
  for (int s = s0; s < s1; s += kGenericRows) {
    int64_t toks[kGenericRows];
    bool ok[kGenericRows];
#pragma unroll
    for (int u = 0; u < kGenericRows; ++u) {
      int64_t tk = 0;
      const bool found = slot_token_of(get_id, s + u < s1 ? s + u : s1 - 1, chunk, chunk_shift, seq_len, tk);
      ok[u] = s + u < s1 && found;
      toks[u] = ok[u] ? tk : 0;
    }
#pragma unroll
    for (int u = 0; u < kGenericRows; ++u) asm volatile("" : "+v"(toks[u]));
    T kr[kGenericRows][J], vr[kGenericRows][J];
#pragma unroll
    for (int u = 0; u < kGenericRows; ++u)
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int d = lane + kWave * j;
        const int64_t off = toks[u] * D + (d < D ? d : 0);
        kr[u][j] = load_global_elem<T>(kb + off);
        vr[u][j] = load_global_elem<T>(vb + off);
      }
    __builtin_amdgcn_sched_barrier(0);
    float sc[kGenericRows];
#pragma unroll
    for (int u = 0; u < kGenericRows; ++u) {
      float dot = 0.f;
#pragma unroll
      for (int j = 0; j < J; ++j)
        if (lane + kWave * j < D) dot = fmaf(qf[j], to_f32(kr[u][j]), dot);
      sc[u] = dot;
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
      for (int u = 0; u < kGenericRows; ++u) sc[u] += xor_lanes(sc[u], off);
    float mb = -INFINITY;
#pragma unroll
    for (int u = 0; u < kGenericRows; ++u) {
      sc[u] = ok[u] ? sc[u] : -INFINITY;
      mb = fmaxf(mb, sc[u]);
    }
    if (mb == -INFINITY) continue;  // no live slot in the batch (uniform)
    const float m_new = fmaxf(m, mb);
    const float alpha = fast_exp2(m - m_new);
    float pr[kGenericRows];
    float psum = 0.f;
#pragma unroll
    for (int u = 0; u < kGenericRows; ++u) {
      pr[u] = fast_exp2(sc[u] - m_new);
      psum += pr[u];
    }
    l = l * alpha + psum;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float x = acc[j] * alpha;
#pragma unroll
      for (int u = 0; u < kGenericRows; ++u) x = fmaf(pr[u], lane + kWave * j < D ? to_f32(vr[u][j]) : 0.f, x);
      acc[j] = x;
    }
    m = m_new;
  }
  const int64_t p = bh * num_tiles + t;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int d = lane + kWave * j;
    if (d < D) part_acc[p * D + d] = acc[j];
  }
  if (lane == 0) {
    part_ml[2 * p] = m;
    part_ml[2 * p + 1] = l;
  }
}

constexpr int kMergeRows = 64;  // partial rows per thread in the one-round-trip merge

// Block-wide reductions for 256-thread blocks.
__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, xor_lanes(v, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  return v;
}
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  v = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return v;
}

// Log-sum-exp merge of the split partials of one (b,h) (the merge pass of
// csrc/csa_attention.cu:224-274): M = max m_t, L = sum_{l_t>0} l_t 2^(m_t-M),
// out = sum_{l_t>0} 2^(m_t-M) acc_t / L, or 0 when L is not positive.
// 256 threads; the tile loops carry no data-dependent branches, so their loads
// issue back to back.  Column d is summed by G = max(1, 256 / D) thread groups.
template <typename T>
__global__ __launch_bounds__(256) void csa_merge_kernel(const float* __restrict__ part_ml,
                                                        const float* __restrict__ part_acc,
                                                        T* __restrict__ out, int D, int num_tiles) {
  __shared__ float red[4];
  __shared__ float colsum[256];
  __shared__ float wts[256];
  const int64_t bh = blockIdx.x;
  const float* ml = part_ml + 2 * bh * num_tiles;
  const float* pa = part_acc + bh * num_tiles * static_cast<int64_t>(D);
  const int tid = threadIdx.x;
  if (D <= 256 && num_tiles <= 256 && num_tiles <= kMergeRows * (256 / D)) {
    // One memory round trip: every thread requests its column of each of its
    // partial rows and (m, l) of tile `tid` before anything waits; the tile
    // weights then meet in LDS.
    const int G = 256 / D, g = tid / D, d = tid - g * D;
    float x[kMergeRows];
#pragma unroll
    for (int i = 0; i < kMergeRows; ++i) {
      const int t = g + i * G;
      x[i] = (g < G && t < num_tiles) ? pa[static_cast<int64_t>(t) * D + d] : 0.f;
    }
    const float mt = tid < num_tiles ? ml[2 * tid] : -INFINITY;
    const float lt = tid < num_tiles ? ml[2 * tid + 1] : 0.f;
    const float M = block_max256(lt > 0.f ? mt : -INFINITY, red);
    const float w = (lt > 0.f && M != -INFINITY) ? fast_exp2(mt - M) : 0.f;
    wts[tid] = w;
    const float Lt = block_sum256(w * lt, red);  // its barriers also publish wts
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < kMergeRows; ++i) {
      const int t = g + i * G;
      if (g < G && t < num_tiles) a = fmaf(wts[t], x[i], a);
    }
    colsum[tid] = a;
    __syncthreads();
    if (tid < D) {
      float o = 0.f;
      for (int j = 0; j < G; ++j) o += colsum[j * D + tid];
      out[bh * D + tid] = from_f32<T>(Lt > 0.f ? o / Lt : 0.f);
    }
    return;
  }
  float mx = -INFINITY;
  for (int t = threadIdx.x; t < num_tiles; t += 256) mx = fmaxf(mx, ml[2 * t]);
  mx = block_max256(mx, red);
  float L = 0.f;
  if (mx != -INFINITY) {
    for (int t = threadIdx.x; t < num_tiles; t += 256) {
      const float lt = ml[2 * t + 1];
      L += lt > 0.f ? lt * fast_exp2(ml[2 * t] - mx) : 0.f;
    }
  }
  L = block_sum256(L, red);
  const float inv = (mx != -INFINITY && L > 0.f) ? 1.f / L : 0.f;
  const int G = D >= 256 ? 1 : 256 / D;
  const int g = threadIdx.x / (D >= 256 ? 256 : D);
  for (int d0 = 0; d0 < D; d0 += (D >= 256 ? 256 : D)) {
    const int d = d0 + threadIdx.x % (D >= 256 ? 256 : D);
    float a = 0.f;
    if (g < G && d < D && inv > 0.f) {
#pragma unroll 8
      for (int t = g; t < num_tiles; t += G) {
        const float lt = ml[2 * t + 1];
        const float w = lt > 0.f ? fast_exp2(ml[2 * t] - mx) : 0.f;
        a = fmaf(w, pa[static_cast<int64_t>(t) * D + d], a);
      }
    }
    if (G > 1) {
      colsum[threadIdx.x] = a;
      __syncthreads();
      if (g == 0 && d < D) {
        for (int j = 1; j < G; ++j) a += colsum[threadIdx.x + j * D];
        out[bh * D + d] = from_f32<T>(a * inv);
      }
      __syncthreads();
    } else if (d < D) {
      out[bh * D + d] = from_f32<T>(a * inv);
    }
  }
}

// Merge of at most kMergeColTiles partials per head, spread over workgroups
// of (head, kMergeCols output columns): 256 threads = kMergeCols columns x 8
// tile groups.  Every load -- the thread's tiles of its column, and lane l's
// (m, l) of tile l -- is one unconditional batch; each wavefront forms the
// tile weights itself (a wavefront max and sum over the tiles, one tile per
// lane) and a thread takes its tiles' weights by lane shuffle, so the only
// barrier is the one that sums the 8 tile groups of a column.
constexpr int kMergeColTiles = kWave;
constexpr int kMergeCols = 32;
constexpr int kMergeGroups = 256 / kMergeCols;  // 8

template <typename T>
__global__ __launch_bounds__(256) void csa_merge_cols_kernel(const float* __restrict__ part_ml,
                                                             const float* __restrict__ part_acc,
                                                             T* __restrict__ out, int D, int num_tiles,
                                                             int col_blocks) {
  constexpr int TPG = kMergeColTiles / kMergeGroups;  // tiles per group
  __shared__ float colsum[256];
  const int tid = threadIdx.x, lane = tid % kWave;
  const int64_t bh = blockIdx.x / col_blocks;
  const int cb = static_cast<int>(blockIdx.x - bh * col_blocks);
  const int cl = tid % kMergeCols, g = tid / kMergeCols;
  const int d = cb * kMergeCols + cl;
  const float* ml = part_ml + 2 * bh * num_tiles;
  const float* pa = part_acc + bh * num_tiles * static_cast<int64_t>(D) + (d < D ? d : 0);
  float x[TPG];
#pragma unroll
  for (int i = 0; i < TPG; ++i) {
    const int t = g + kMergeGroups * i;
    x[i] = load_global_raw<float>(pa + static_cast<int64_t>(t < num_tiles ? t : 0) * D);
  }
  const uint2 mlr = load_global_u2(ml + 2 * (lane < num_tiles ? lane : 0));
  const float mt = __uint_as_float(mlr.x), lt = lane < num_tiles ? __uint_as_float(mlr.y) : 0.f;
  float M = lt > 0.f ? mt : -INFINITY;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, xor_lanes(M, off));
  const float w = (lt > 0.f && M != -INFINITY) ? fast_exp2(mt - M) : 0.f;
  const float L = wave_sum(w * lt);
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < TPG; ++i) {
    const int t = g + kMergeGroups * i;
    const float wt = __shfl(w, t < kWave ? t : 0, kWave);
    a = fmaf(t < num_tiles ? wt : 0.f, x[i], a);
  }
  colsum[tid] = a;
  __syncthreads();
  if (tid < kMergeCols && d < D) {
    float o = 0.f;
#pragma unroll
    for (int j = 0; j < kMergeGroups; ++j) o += colsum[j * kMergeCols + tid];
    out[bh * D + d] = from_f32<T>(L > 0.f ? o / L : 0.f);
  }
}

// ---------------------------------------------------------------------------
// Chunk summaries (chunk_mean, hybrid_attention/reference.py:40-45).
// ---------------------------------------------------------------------------
// Chunk a summary workgroup computes: chunk_begin + its index in the request,
// or, with token_pos set (one workgroup per head), the chunk that the token at
// *token_pos completes; -1 when that token completes no chunk that both the
// cache and the summary hold (the workgroup then does nothing).
__device__ __forceinline__ int64_t summary_chunk(const int64_t* token_pos, int64_t chunk_begin, int64_t nreq,
                                                 int chunk, int64_t seq_len, int64_t summary_chunks) {
  if (token_pos == nullptr) return chunk_begin + blockIdx.x % nreq;
  const int64_t pos = *token_pos;
  if (pos < 0 || (pos + 1) % chunk != 0) return -1;
  const int64_t c = pos / chunk;
  return (c < summary_chunks && (c + 1) * chunk <= seq_len) ? c : -1;
}

template <typename T, int D>
__global__ __launch_bounds__(64) void csa_summary_vec_kernel(const T* __restrict__ k,
                                                             float* __restrict__ summary,
                                                             int64_t seq_len, int chunk,
                                                             int64_t summary_chunks,
                                                             int64_t chunk_begin, int64_t nreq,
                                                             const int64_t* __restrict__ token_pos) {
  using L = AttendLayout<T, D>;
  constexpr int VEC = L::VEC, LPR = L::LPR, RPL = L::RPL;
  const int lane = threadIdx.x;
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int64_t bh = blockIdx.x / nreq;
  const int64_t c = summary_chunk(token_pos, chunk_begin, nreq, chunk, seq_len, summary_chunks);
  if (c < 0) return;
  const T* __restrict__ base = k + (bh * seq_len + c * chunk) * D + col * VEC;
  float acc[VEC];
  // 16 rows per lane per batch (measured, B4 H8 S32768 chunk 64: 47.5-48.0
  // against 50.3 us with 4; B1 level)
  wave_chunk_colsum<T, D, 16>(base, chunk, grp, acc);
  if (grp == 0) {
    float* dst = summary + (bh * summary_chunks + c) * D + col * VEC;
    const float fc = static_cast<float>(chunk);
#pragma unroll
    for (int e = 0; e < VEC; ++e) dst[e] = acc[e] / fc;
  }
}

template <typename T>
__global__ __launch_bounds__(64) void csa_summary_generic_kernel(
    const T* __restrict__ k, float* __restrict__ summary, int64_t seq_len, int D, int chunk,
    int64_t summary_chunks, int64_t chunk_begin, int64_t nreq, const int64_t* __restrict__ token_pos) {
  const int64_t bh = blockIdx.x / nreq;
  const int64_t c = summary_chunk(token_pos, chunk_begin, nreq, chunk, seq_len, summary_chunks);
  if (c < 0) return;
  const T* __restrict__ base = k + (bh * seq_len + c * chunk) * D;
  const float fc = static_cast<float>(chunk);
  for (int d = threadIdx.x; d < D; d += kWave) {
    float a = 0.f;
    for (int r = 0; r < chunk; ++r) a += to_f32(base[static_cast<int64_t>(r) * D + d]);
    summary[(bh * summary_chunks + c) * D + d] = a / fc;
  }
}

// ---------------------------------------------------------------------------
// Chunk scores -> order keys of score[c] = (q . summary[c]) * scale
// (reference.py:54-55).  Summary rows are fp32: a lane loads 4 columns; R rows
// per wavefront.
// ---------------------------------------------------------------------------
template <typename T, int D, int R>
__global__ __launch_bounds__(64) void csa_score_vec_kernel(const T* __restrict__ q,
                                                           const float* __restrict__ summary,
                                                           uint32_t* __restrict__ keys, int64_t C,
                                                           int64_t blocks_per_head, float scale) {
  constexpr int LPR = D / 4;
  constexpr int RPL = kWave / LPR;
  static_assert(R % RPL == 0, "R must be a multiple of rows per load");
  constexpr int U = R / RPL;
  const int lane = threadIdx.x;
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int64_t bh = blockIdx.x / blocks_per_head;
  const int64_t c0 = (blockIdx.x % blocks_per_head) * R;
  // One memory round trip: the summary rows are requested unconditionally
  // (rows past C re-read row c0; their scores are never stored), then q, and
  // only then is anything consumed.
  const float* __restrict__ sb = summary + bh * C * D + col * 4;
  uint4 rs[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t c = c0 + grp + RPL * u;
    rs[u] = load_global_u4(sb + (c < C ? c : c0) * D);
  }
  float qf[4];
  load4_f32<T>(q + bh * D + col * 4, qf);
  float sc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float r4[4];
    widen16<float>(rs[u], r4);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) d = fmaf(qf[e], r4[e], d);
    sc[u] = d;
  }
  // Transposed row sums (the bits of a butterfly per row; one key store per
  // row from the lane that holds it).
  static_assert(U <= LPR && (U & (U - 1)) == 0, "one summed row per lane group of LPR / U lanes");
  const float ssum = transposed_group_sum<U, LPR>(sc);
  if (col % (LPR / U) == 0) {
    const int64_t c = c0 + grp + RPL * (col / (LPR / U));
    if (c < C) keys[bh * C + c] = order_key(ssum * scale);
  }
}

template <typename T>
__global__ __launch_bounds__(64) void csa_score_generic_kernel(const T* __restrict__ q,
                                                               const float* __restrict__ summary,
                                                               uint32_t* __restrict__ keys, int64_t C,
                                                               int D, float scale) {
  const int64_t bh = blockIdx.x / C;
  const int64_t c = blockIdx.x % C;
  float d = 0.f;
  for (int j = threadIdx.x; j < D; j += kWave)
    d = fmaf(to_f32(q[bh * D + j]), summary[(bh * C + c) * D + j], d);
  d = wave_sum(d);
  if (threadIdx.x == 0) keys[bh * C + c] = order_key(d * scale);
}

// Top-k per (b,h): keys -> LDS in one batch of loads (when they fit), then the
// wavefront top-k of csa_device.hpp (register path of M keys per lane, or the
// radix select).
template <int M, bool kInLds>
__global__ __launch_bounds__(64) void csa_topk_kernel(const uint32_t* __restrict__ keys,
                                                      int32_t* __restrict__ out, int64_t C, int k) {
  extern __shared__ uint64_t lds64[];
  uint32_t* scratch = reinterpret_cast<uint32_t*>(lds64);
  uint32_t* hist = scratch + kTopkScratchWords;
  uint32_t* skey = hist + 256;
  int32_t* sidx = reinterpret_cast<int32_t*>(skey + k);
  uint32_t* counter = reinterpret_cast<uint32_t*>(sidx + k);
  uint32_t* kl = counter + 1;
  const int64_t bh = blockIdx.x;
  const uint32_t* kg = keys + bh * C;
  int32_t* o = out + bh * k;
  auto emit = [&](int r, int32_t i) { o[r] = i; };
  if constexpr (kInLds) {
    for (int i = threadIdx.x; i < C; i += kWave) kl[i] = kg[i];
    wave_lds_sync();
    wave_topk<M>(kl, static_cast<int>(C), k, scratch, hist, skey, sidx, counter, emit);
  } else {
    wave_topk<M>(kg, static_cast<int>(C), k, scratch, hist, skey, sidx, counter, emit);
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int kMaxTopkSelect = 4096;  // LDS bound of csa_topk_kernel
constexpr size_t kLdsBudget = 64 * 1024;

int chunk_shift_of(int64_t chunk) {
  if (chunk > 0 && (chunk & (chunk - 1)) == 0) {
    int s = 0;
    while ((int64_t{1} << s) < chunk) ++s;
    return s;
  }
  return -1;
}

size_t decode_ws_bytes(int64_t bh, int64_t D, int64_t tiles) {
  const size_t ml = static_cast<size_t>(bh * tiles * 2) * sizeof(float);
  const size_t ml_al = (ml + 255) & ~size_t{255};
  return ml_al + static_cast<size_t>(bh * tiles * D) * sizeof(float);
}

template <typename T, typename IdxT>
int launch_attend(const void* q, const void* k, const void* v, const void* idx, float* part_ml,
                  float* part_acc, int64_t bh, int64_t S, int64_t D, int top_k, int chunk,
                  int tile, int num_tiles, hipStream_t stream) {
  const float qscale = kLog2e / sqrtf(static_cast<float>(D));
  const int cshift = chunk_shift_of(chunk);
  const dim3 grid(static_cast<uint32_t>(bh * num_tiles));
  const T* qp = static_cast<const T*>(q);
  const T* kp = static_cast<const T*>(k);
  const T* vp = static_cast<const T*>(v);
  const IdxT* ip = static_cast<const IdxT*>(idx);
  constexpr int VEC = Vec16<T>::N;
  const bool aligned = (reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) |
                        reinterpret_cast<uintptr_t>(v)) % 16 == 0;
#define CSAHCA_ATTEND_VEC(DD)                                                                  \
  if (aligned && D == DD && (DD / VEC) <= kWave) {                                           \
    return launch("csa_attend_vec_kernel",                                                   \
                  csa_attend_vec_kernel<T, IdxT, (DD / VEC <= kWave ? DD : VEC), 4>, grid,   \
                  dim3(kWave), 0, stream, ip, S, kp, vp, qp, num_tiles, top_k, tile, chunk,    \
                  part_ml, part_acc, qscale);                                                \
  }
  CSAHCA_ATTEND_VEC(64)
  CSAHCA_ATTEND_VEC(128)
  CSAHCA_ATTEND_VEC(256)
  CSAHCA_ATTEND_VEC(512)
#undef CSAHCA_ATTEND_VEC
  const int64_t J = ceil_div(D, kWave);
#define CSAHCA_ATTEND_GEN(JJ)                                                                  \
  if (J <= JJ) {                                                                               \
    return launch("csa_attend_generic_kernel", csa_attend_generic_kernel<T, IdxT, JJ>, grid,   \
                  dim3(kWave), 0, stream, qp, kp, vp, ip, part_ml, part_acc, S,                \
                  static_cast<int>(D), top_k, chunk, cshift, tile, num_tiles, qscale);         \
  }
  CSAHCA_ATTEND_GEN(1)
  CSAHCA_ATTEND_GEN(2)
  CSAHCA_ATTEND_GEN(4)
  CSAHCA_ATTEND_GEN(8)
  CSAHCA_ATTEND_GEN(16)
#undef CSAHCA_ATTEND_GEN
  return fail(CSAHCA_ERR_ARGUMENT, "head_dim > 1024 is not supported");
}

int csa_decode_impl(const void* q, const void* k, const void* v, const void* idx, void* out,
                    int dtype, int index_dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                    int64_t top_k, int64_t chunk, int64_t tile, const char* d_msg,
                    void* workspace, size_t workspace_bytes, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(valid_dtype(dtype), "q, k_cache and v_cache must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(index_dtype == CSAHCA_I32 || index_dtype == CSAHCA_I64,
                 "chunk_indices must be int32 or int64");
  CSAHCA_REQUIRE(B >= 0 && H >= 0 && S >= 0 && D >= 0 && top_k >= 0, "negative dimension");
  CSAHCA_REQUIRE(chunk > 0, "chunk_size must be positive");
  CSAHCA_REQUIRE(tile > 0, "tile_size must be positive");
  CSAHCA_REQUIRE(D <= 1024, d_msg);
  CSAHCA_REQUIRE(chunk <= INT_MAX && top_k <= INT_MAX, "chunk_size and top_k must fit in int32");
  CSAHCA_REQUIRE(top_k * chunk <= INT_MAX, "top_k * chunk_size must fit in int32");
  const int64_t bh = B * H;
  if (bh == 0 || D == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(q && out && (S == 0 || (k && v)) && (idx || top_k == 0), "null tensor pointer");
  const int64_t total = top_k * chunk;
  const int64_t tiles = std::max<int64_t>(1, ceil_div(total, tile));
  CSAHCA_REQUIRE(bh * tiles <= INT32_MAX, "too many split-KV work items");
  const size_t need = decode_ws_bytes(bh, D, tiles);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CSAHCA_ERR_WORKSPACE, "workspace too small for csa decode");
  float* part_ml = static_cast<float*>(workspace);
  const size_t ml = static_cast<size_t>(bh * tiles * 2) * sizeof(float);
  float* part_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + ((ml + 255) & ~size_t{255}));
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const int tl = static_cast<int>(std::min<int64_t>(tile, std::max<int64_t>(total, 1)));
  // Stand-ins for pointers that are never dereferenced (no selected slots / no tokens).
  const void* idx_ok = idx ? idx : q;
  const void* k_ok = k ? k : q;
  const void* v_ok = v ? v : q;
  return dispatch_dtype(dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    int rc = index_dtype == CSAHCA_I32
                 ? launch_attend<T, int32_t>(q, k_ok, v_ok, idx_ok, part_ml, part_acc, bh, S, D,
                                             static_cast<int>(top_k), static_cast<int>(chunk), tl,
                                             static_cast<int>(tiles), stream)
                 : launch_attend<T, int64_t>(q, k_ok, v_ok, idx_ok, part_ml, part_acc, bh, S, D,
                                             static_cast<int>(top_k), static_cast<int>(chunk), tl,
                                             static_cast<int>(tiles), stream);
    if (rc != CSAHCA_OK) return rc;
    if (tiles <= kMergeColTiles) {
      const int64_t cbs = ceil_div(D, kMergeCols);
      return launch("csa_merge_cols_kernel", csa_merge_cols_kernel<T>, dim3(static_cast<uint32_t>(bh * cbs)),
                    dim3(256), 0, stream, static_cast<const float*>(part_ml), static_cast<const float*>(part_acc),
                    static_cast<T*>(out), static_cast<int>(D), static_cast<int>(tiles), static_cast<int>(cbs));
    }
    return launch("csa_merge_kernel", csa_merge_kernel<T>, dim3(static_cast<uint32_t>(bh)), dim3(256), 0,
                  stream, static_cast<const float*>(part_ml), static_cast<const float*>(part_acc),
                  static_cast<T*>(out), static_cast<int>(D), static_cast<int>(tiles));
  });
}

}  // namespace

// Shared with csa_step.hip: scores + top-k into out_indices using `keys` scratch.
int csa_select_launch(const void* q, const float* summary, int32_t* out_indices, int dtype,
                      int64_t bh, int64_t C, int64_t D, int64_t k, uint32_t* keys,
                      hipStream_t stream) {
  const float scale = 1.0f / sqrtf(static_cast<float>(D));
  const bool aligned = (reinterpret_cast<uintptr_t>(summary) | reinterpret_cast<uintptr_t>(q)) % 16 == 0;
  int rc = dispatch_dtype(dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    const T* qp = static_cast<const T*>(q);
#define CSAHCA_SCORE_VEC(DD, RR)                                                           \
  if (aligned && D == DD) {                                                                \
    const int64_t bph = ceil_div(C, RR);                                                   \
    return launch("csa_score_vec_kernel", csa_score_vec_kernel<T, DD, RR>,                 \
                  dim3(static_cast<uint32_t>(bh * bph)), dim3(kWave), 0, stream, qp,       \
                  summary, keys, C, bph, scale);                                           \
  }
    CSAHCA_SCORE_VEC(64, 16)
    CSAHCA_SCORE_VEC(128, 16)
    CSAHCA_SCORE_VEC(256, 8)
#undef CSAHCA_SCORE_VEC
    return launch("csa_score_generic_kernel", csa_score_generic_kernel<T>,
                  dim3(static_cast<uint32_t>(bh * C)), dim3(kWave), 0, stream, qp, summary, keys, C,
                  static_cast<int>(D), scale);
  });
  if (rc != CSAHCA_OK) return rc;
  const size_t base = kCandBytes + (256 + 2 * static_cast<size_t>(k) + 1) * sizeof(uint32_t);
  const bool in_lds = base + static_cast<size_t>(C) * sizeof(uint32_t) <= kLdsBudget;
  const size_t lds = base + (in_lds ? static_cast<size_t>(C) * sizeof(uint32_t) : 0);
  const dim3 grid(static_cast<uint32_t>(bh));
  const uint32_t* kp = keys;
  const int ki = static_cast<int>(k);
  switch (topk_regs_for(C, k) * 2 + (in_lds ? 1 : 0)) {
    case 17: return launch("csa_topk_kernel", csa_topk_kernel<8, true>, grid, dim3(kWave), lds, stream, kp, out_indices, C, ki);
    case 65: return launch("csa_topk_kernel", csa_topk_kernel<32, true>, grid, dim3(kWave), lds, stream, kp, out_indices, C, ki);
    case 1: return launch("csa_topk_kernel", csa_topk_kernel<0, true>, grid, dim3(kWave), lds, stream, kp, out_indices, C, ki);
    default: return launch("csa_topk_kernel", csa_topk_kernel<0, false>, grid, dim3(kWave), lds, stream, kp, out_indices, C, ki);
  }
}

}  // namespace csahca

using namespace csahca;

extern "C" int64_t csahca_csa_auto_tile_size(int64_t batch, int64_t heads, int64_t top_k,
                                             int64_t chunk_size) {
  // Aim for ~2048 wavefronts (8 per CU on 256 CUs) while keeping >= 16 slots
  // per wavefront, so each work item moves at least 16 K rows + 16 V rows.
  const int64_t total = std::max<int64_t>(1, top_k * chunk_size);
  const int64_t bh = std::max<int64_t>(1, batch * heads);
  const int64_t want_tiles = std::max<int64_t>(1, ceil_div(2048, bh));
  const int64_t max_tiles = std::max<int64_t>(1, ceil_div(total, 16));
  const int64_t tiles = std::min(want_tiles, max_tiles);
  return std::max<int64_t>(1, ceil_div(total, tiles));
}

extern "C" size_t csahca_csa_decode_workspace_bytes(int64_t batch, int64_t heads,
                                                    int64_t head_dim, int64_t top_k,
                                                    int64_t chunk_size, int64_t tile_size) {
  if (batch < 0 || heads < 0 || head_dim < 0 || top_k < 0 || chunk_size <= 0) return 0;
  if (tile_size <= 0) tile_size = csahca_csa_auto_tile_size(batch, heads, top_k, chunk_size);
  const int64_t tiles = std::max<int64_t>(1, ceil_div(top_k * chunk_size, tile_size));
  return decode_ws_bytes(batch * heads, head_dim, tiles);
}

extern "C" int csahca_csa_decode_forward(const void* q, const void* k_cache, const void* v_cache,
                                         const void* chunk_indices, void* out, int dtype,
                                         int index_dtype, int64_t batch, int64_t heads,
                                         int64_t seq_len, int64_t head_dim, int64_t top_k,
                                         int64_t chunk_size, void* workspace,
                                         size_t workspace_bytes, void* stream) {
  const int64_t tile = chunk_size > 0 ? csahca_csa_auto_tile_size(batch, heads, top_k, chunk_size) : 1;
  return csa_decode_impl(q, k_cache, v_cache, chunk_indices, out, dtype, index_dtype, batch,
                         heads, seq_len, head_dim, top_k, chunk_size, tile,
                         "head_dim > 1024 is not supported by the v1 kernel", workspace,
                         workspace_bytes, stream);
}

extern "C" int csahca_csa_decode_forward_tiled(const void* q, const void* k_cache,
                                               const void* v_cache, const void* chunk_indices,
                                               void* out, int dtype, int index_dtype,
                                               int64_t batch, int64_t heads, int64_t seq_len,
                                               int64_t head_dim, int64_t top_k,
                                               int64_t chunk_size, int64_t tile_size,
                                               void* workspace, size_t workspace_bytes,
                                               void* stream) {
  return csa_decode_impl(q, k_cache, v_cache, chunk_indices, out, dtype, index_dtype, batch,
                         heads, seq_len, head_dim, top_k, chunk_size, tile_size,
                         "head_dim > 1024 is not supported by the tiled kernel", workspace,
                         workspace_bytes, stream);
}

namespace {

// Launches the summary kernels over num_chunks chunks from chunk_begin, or,
// with token_pos set (num_chunks = 1), over the chunk *token_pos completes.
int chunk_summary_launch(const void* k_cache, float* summary, int dtype, int64_t batch, int64_t heads,
                         int64_t seq_len, int64_t head_dim, int64_t chunk_size, int64_t summary_chunks,
                         int64_t chunk_begin, int64_t num_chunks, const int64_t* token_pos,
                         void* stream_ptr) {
  const int64_t bh = batch * heads;
  if (bh == 0 || num_chunks == 0 || head_dim == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(k_cache && summary, "null tensor pointer");
  CSAHCA_REQUIRE(bh * num_chunks <= INT32_MAX, "too many chunks in one call");
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const dim3 grid(static_cast<uint32_t>(bh * num_chunks));
  const bool aligned = (reinterpret_cast<uintptr_t>(k_cache) % 16 == 0) &&
                       (reinterpret_cast<uintptr_t>(summary) % 16 == 0);
  return dispatch_dtype(dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    const T* kp = static_cast<const T*>(k_cache);
    constexpr int VEC = Vec16<T>::N;
#define CSAHCA_SUM_VEC(DD)                                                                   \
  if (aligned && head_dim == DD && DD / VEC <= kWave) {                                      \
    return launch("csa_summary_vec_kernel",                                                  \
                  csa_summary_vec_kernel<T, (DD / VEC <= kWave ? DD : VEC)>, grid,           \
                  dim3(kWave), 0, stream, kp, summary, seq_len,                              \
                  static_cast<int>(chunk_size), summary_chunks, chunk_begin, num_chunks,     \
                  token_pos);                                                                \
  }
    CSAHCA_SUM_VEC(64)
    CSAHCA_SUM_VEC(128)
    CSAHCA_SUM_VEC(256)
    CSAHCA_SUM_VEC(512)
#undef CSAHCA_SUM_VEC
    return launch("csa_summary_generic_kernel", csa_summary_generic_kernel<T>, grid, dim3(kWave),
                  0, stream, kp, summary, seq_len, static_cast<int>(head_dim),
                  static_cast<int>(chunk_size), summary_chunks, chunk_begin, num_chunks, token_pos);
  });
}

int check_summary_args(int dtype, int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                       int64_t chunk_size) {
  CSAHCA_REQUIRE(valid_dtype(dtype), "k_cache must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(batch >= 0 && heads >= 0 && seq_len >= 0 && head_dim >= 0, "negative dimension");
  CSAHCA_REQUIRE(chunk_size > 0 && chunk_size <= INT_MAX, "chunk_size must be positive");
  CSAHCA_REQUIRE(head_dim <= 1024, "head_dim > 1024 is not supported");
  return CSAHCA_OK;
}

}  // namespace

extern "C" int csahca_csa_chunk_summary(const void* k_cache, float* summary, int dtype,
                                        int64_t batch, int64_t heads, int64_t seq_len,
                                        int64_t head_dim, int64_t chunk_size,
                                        int64_t summary_chunks, int64_t chunk_begin,
                                        int64_t num_chunks, void* stream_ptr) {
  clear_error();
  const int rc = check_summary_args(dtype, batch, heads, seq_len, head_dim, chunk_size);
  if (rc != CSAHCA_OK) return rc;
  CSAHCA_REQUIRE(chunk_begin >= 0 && num_chunks >= 0, "chunk range must be non-negative");
  CSAHCA_REQUIRE((chunk_begin + num_chunks) * chunk_size <= seq_len,
                 "requested chunks extend past seq_len (only complete chunks have summaries)");
  CSAHCA_REQUIRE(summary_chunks >= chunk_begin + num_chunks, "summary has too few chunk rows");
  return chunk_summary_launch(k_cache, summary, dtype, batch, heads, seq_len, head_dim, chunk_size,
                              summary_chunks, chunk_begin, num_chunks, nullptr, stream_ptr);
}

extern "C" int csahca_csa_chunk_summary_at(const void* k_cache, float* summary, int dtype, int64_t batch,
                                           int64_t heads, int64_t seq_len, int64_t head_dim,
                                           int64_t chunk_size, int64_t summary_chunks,
                                           const int64_t* token_pos, void* stream_ptr) {
  clear_error();
  const int rc = check_summary_args(dtype, batch, heads, seq_len, head_dim, chunk_size);
  if (rc != CSAHCA_OK) return rc;
  CSAHCA_REQUIRE(summary_chunks >= 0, "negative dimension");
  CSAHCA_REQUIRE(token_pos != nullptr || batch * heads == 0, "null token_pos pointer");
  if (summary_chunks == 0) return CSAHCA_OK;
  return chunk_summary_launch(k_cache, summary, dtype, batch, heads, seq_len, head_dim, chunk_size,
                              summary_chunks, 0, 1, token_pos, stream_ptr);
}

extern "C" size_t csahca_csa_select_workspace_bytes(int64_t batch, int64_t heads,
                                                    int64_t num_chunks) {
  if (batch < 0 || heads < 0 || num_chunks < 0) return 0;
  return static_cast<size_t>(batch * heads * num_chunks) * sizeof(uint32_t);
}

extern "C" int csahca_csa_select_topk(const void* q, const float* summary, int32_t* out_indices,
                                      int dtype, int64_t batch, int64_t heads, int64_t num_chunks,
                                      int64_t head_dim, int64_t top_k, void* workspace,
                                      size_t workspace_bytes, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(valid_dtype(dtype), "q must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(batch >= 0 && heads >= 0 && num_chunks >= 0 && head_dim >= 0,
                 "negative dimension");
  CSAHCA_REQUIRE(top_k >= 0, "top_k must be non-negative");
  CSAHCA_REQUIRE(head_dim <= 1024, "head_dim > 1024 is not supported");
  const int64_t k = std::min(top_k, num_chunks);
  CSAHCA_REQUIRE(k <= kMaxTopkSelect, "top_k > 4096 is not supported by the selection kernel");
  CSAHCA_REQUIRE(num_chunks <= INT_MAX, "num_chunks must fit in int32");
  const int64_t bh = batch * heads;
  if (bh == 0 || k == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(q && summary && out_indices, "null tensor pointer");
  CSAHCA_REQUIRE(bh * num_chunks <= INT32_MAX, "too many chunks in one call");
  const size_t need = csahca_csa_select_workspace_bytes(batch, heads, num_chunks);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CSAHCA_ERR_WORKSPACE, "workspace too small for csa select");
  return csa_select_launch(q, summary, out_indices, dtype, bh, num_chunks, head_dim, k,
                           static_cast<uint32_t*>(workspace), static_cast<hipStream_t>(stream_ptr));
}
