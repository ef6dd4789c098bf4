// csa.hip -- CSA decode kernels for gfx950 and their C-ABI entry points.
//
// Decode step (one query token per (batch, head)):
//   1. csa_summary_*   : fp32 mean of every chunk of K (the chunk summaries).
//   2. csa_score_*     : score[c] = (q . summary[c]) / sqrt(D), fp32.
//   3. csa_topk_kernel : per (b,h) one wavefront selects the top-k chunks by
//                        radix select over order-preserving uint32 keys, then
//                        ranks the k winners (score desc, chunk id asc).
//   4. csa_attend_*    : split-KV sparse attention.  Work item = one wavefront
//                        over `tile` consecutive selected-token slots of one
//                        (b,h); K/V rows are fetched with 16-byte lane loads so
//                        a wavefront-wide load moves whole 256-byte rows
//                        (D=128, bf16); online softmax in registers; writes an
//                        fp32 partial (m, l, acc[D]).
//   5. csa_merge_kernel: log-sum-exp merge of the partials of each (b,h).
// All offsets are 64-bit.
#include "common.hpp"

#include <climits>

namespace csahca {
namespace {

// ---------------------------------------------------------------------------
// Selected-slot -> token mapping shared by the attend kernels.
// Slot s of (b,h) is token idx[s / chunk] * chunk + s % chunk; the slot is
// skipped when the chunk id is negative or the token is past seq_len
// (csrc/csa_attention.cu:176-185).
// ---------------------------------------------------------------------------
template <typename IdxT>
__device__ __forceinline__ bool slot_token(const IdxT* __restrict__ ib, int s, int chunk,
                                           int chunk_shift, int64_t seq_len, int64_t& tok) {
  int cs, off;
  if (chunk_shift >= 0) {
    cs = s >> chunk_shift;
    off = s & (chunk - 1);
  } else {
    cs = s / chunk;
    off = s - cs * chunk;
  }
  const int64_t c = static_cast<int64_t>(ib[cs]);
  tok = c * chunk + off;
  return c >= 0 && tok < seq_len;
}

// ---------------------------------------------------------------------------
// Split-KV sparse attention, vectorised path.
// D = VEC * LPR with LPR (lanes per row) a power of two <= 64; a wavefront-wide
// 16-byte load covers RPL = 64 / LPR rows.  Each lane owns VEC columns of q,
// K, V and acc; a row's dot product is a butterfly over its LPR lanes.
// U row loads per lane per iteration keep 2*U*16 bytes in flight per lane.
// ---------------------------------------------------------------------------
template <typename T, typename IdxT, int D, int U>
__global__ __launch_bounds__(64) void csa_attend_vec_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const IdxT* __restrict__ idx, float* __restrict__ part_ml, float* __restrict__ part_acc,
    int64_t seq_len, int top_k, int chunk, int chunk_shift, int tile, int num_tiles,
    float qscale) {
  constexpr int VEC = Vec16<T>::N;
  constexpr int LPR = D / VEC;
  constexpr int RPL = kWave / LPR;
  static_assert(LPR >= 1 && LPR <= kWave && (LPR & (LPR - 1)) == 0, "bad row split");

  const int lane = threadIdx.x;
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int64_t item = blockIdx.x;
  const int t = static_cast<int>(item % num_tiles);
  const int64_t bh = item / num_tiles;

  float qf[VEC];
  load16<T>(q + bh * D + col * VEC, qf);
#pragma unroll
  for (int e = 0; e < VEC; ++e) qf[e] *= qscale;

  const T* __restrict__ kb = k + bh * seq_len * D + col * VEC;
  const T* __restrict__ vb = v + bh * seq_len * D + col * VEC;
  const IdxT* __restrict__ ib = idx + bh * top_k;
  const int total = top_k * chunk;
  const int s0 = t * tile;
  const int s1 = min(s0 + tile, total);

  float m = -INFINITY, l = 0.f;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;

  for (int base = s0; base < s1; base += RPL * U) {
    float kr[U][VEC], vr[U][VEC];
    bool ok[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int s = base + grp + RPL * u;
      int64_t tok = 0;
      ok[u] = s < s1 && slot_token(ib, s, chunk, chunk_shift, seq_len, tok);
      if (ok[u]) {
        load16<T>(kb + tok * D, kr[u]);
        load16<T>(vb + tok * D, vr[u]);
      } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) kr[u][e] = vr[u][e] = 0.f;
      }
    }
    float sc[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < VEC; ++e) d = fmaf(qf[e], kr[u][e], d);
      sc[u] = d;
    }
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) {
#pragma unroll
      for (int u = 0; u < U; ++u) sc[u] += __shfl_xor(sc[u], off, kWave);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      sc[u] = ok[u] ? sc[u] : -INFINITY;
      mx = fmaxf(mx, sc[u]);
    }
#pragma unroll
    for (int off = LPR; off < kWave; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    const float m_new = fmaxf(m, mx);
    if (m_new == -INFINITY) continue;  // wave-uniform: nothing valid yet
    const float alpha = fast_exp2(m - m_new);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float p = fast_exp2(sc[u] - m_new);
      l += p;
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] = fmaf(p, vr[u][e], acc[e]);
    }
    m = m_new;
  }

  // Fold the RPL row groups (each holds its own rows' l and acc).
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1) {
    l += __shfl_xor(l, off, kWave);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] += __shfl_xor(acc[e], off, kWave);
  }
  const int64_t p = bh * num_tiles + t;
  if (grp == 0) {
    float* dst = part_acc + p * D + col * VEC;
    if constexpr (VEC % 4 == 0) {
#pragma unroll
      for (int e = 0; e < VEC; e += 4)
        *reinterpret_cast<float4*>(dst + e) = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
    } else {
#pragma unroll
      for (int e = 0; e < VEC; ++e) dst[e] = acc[e];
    }
  }
  if (lane == 0) {
    part_ml[2 * p] = m;
    part_ml[2 * p + 1] = l;
  }
}

// Generic path: any D <= 64 * J, any storage type.  Lanes stride the columns
// (coalesced), one row per iteration, wavefront-wide dot reduction.
template <typename T, typename IdxT, int J>
__global__ __launch_bounds__(64) void csa_attend_generic_kernel(
    const T* __restrict__ q, const T* __restrict__ k, const T* __restrict__ v,
    const IdxT* __restrict__ idx, float* __restrict__ part_ml, float* __restrict__ part_acc,
    int64_t seq_len, int D, int top_k, int chunk, int chunk_shift, int tile, int num_tiles,
    float qscale) {
  const int lane = threadIdx.x;
  const int64_t item = blockIdx.x;
  const int t = static_cast<int>(item % num_tiles);
  const int64_t bh = item / num_tiles;
  float qf[J], acc[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int d = lane + kWave * j;
    qf[j] = d < D ? to_f32(q[bh * D + d]) * qscale : 0.f;
    acc[j] = 0.f;
  }
  const T* __restrict__ kb = k + bh * seq_len * D;
  const T* __restrict__ vb = v + bh * seq_len * D;
  const IdxT* __restrict__ ib = idx + bh * top_k;
  const int total = top_k * chunk;
  const int s0 = t * tile;
  const int s1 = min(s0 + tile, total);
  float m = -INFINITY, l = 0.f;
  for (int s = s0; s < s1; ++s) {
    int64_t tok;
    if (!slot_token(ib, s, chunk, chunk_shift, seq_len, tok)) continue;
    const T* kr = kb + tok * D;
    const T* vr = vb + tok * D;
    float dot = 0.f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int d = lane + kWave * j;
      if (d < D) dot = fmaf(qf[j], to_f32(kr[d]), dot);
    }
    dot = wave_sum(dot);
    const float m_new = fmaxf(m, dot);
    const float alpha = fast_exp2(m - m_new);
    const float pr = fast_exp2(dot - m_new);
    l = l * alpha + pr;
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int d = lane + kWave * j;
      const float vv = d < D ? to_f32(vr[d]) : 0.f;
      acc[j] = fmaf(pr, vv, acc[j] * alpha);
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

// Log-sum-exp merge of the split partials of one (b,h) (the merge pass of
// csrc/csa_attention.cu:224-274): M = max m_t, L = sum_{l_t>0} l_t 2^(m_t-M),
// out = sum_{l_t>0} 2^(m_t-M) acc_t / L, or 0 when L is not positive.
template <typename T>
__global__ __launch_bounds__(256) void csa_merge_kernel(const float* __restrict__ part_ml,
                                                        const float* __restrict__ part_acc,
                                                        T* __restrict__ out, int D, int num_tiles) {
  const int64_t bh = blockIdx.x;
  const float* ml = part_ml + 2 * bh * num_tiles;
  __shared__ float s_max, s_inv;
  if (threadIdx.x < kWave) {
    float mx = -INFINITY;
    for (int t = threadIdx.x; t < num_tiles; t += kWave) mx = fmaxf(mx, ml[2 * t]);
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    float L = 0.f;
    for (int t = threadIdx.x; t < num_tiles; t += kWave) {
      const float lt = ml[2 * t + 1];
      if (lt > 0.f) L += lt * fast_exp2(ml[2 * t] - mx);
    }
    L = wave_sum(L);
    if (threadIdx.x == 0) {
      s_max = mx;
      s_inv = L > 0.f ? 1.f / L : 0.f;
    }
  }
  __syncthreads();
  const float mx = s_max, inv = s_inv;
  const float* pa = part_acc + bh * num_tiles * static_cast<int64_t>(D);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float a = 0.f;
    for (int t = 0; t < num_tiles; ++t) {
      const float lt = ml[2 * t + 1];
      if (lt > 0.f) a = fmaf(fast_exp2(ml[2 * t] - mx), pa[static_cast<int64_t>(t) * D + d], a);
    }
    out[bh * D + d] = from_f32<T>(a * inv);
  }
}

// ---------------------------------------------------------------------------
// Chunk summaries (chunk_mean, hybrid_attention/reference.py:40-45).
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(64) void csa_summary_vec_kernel(const T* __restrict__ k,
                                                             float* __restrict__ summary,
                                                             int64_t seq_len, int chunk,
                                                             int64_t summary_chunks,
                                                             int64_t chunk_begin, int64_t nreq) {
  constexpr int VEC = Vec16<T>::N;
  constexpr int LPR = D / VEC;
  constexpr int RPL = kWave / LPR;
  const int lane = threadIdx.x;
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int64_t bh = blockIdx.x / nreq;
  const int64_t c = chunk_begin + blockIdx.x % nreq;
  const T* __restrict__ base = k + (bh * seq_len + c * chunk) * D + col * VEC;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  int r = grp;
  for (; r + 3 * RPL < chunk; r += 4 * RPL) {
    float a[4][VEC];
#pragma unroll
    for (int u = 0; u < 4; ++u) load16<T>(base + static_cast<int64_t>(r + u * RPL) * D, a[u]);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int e = 0; e < VEC; ++e) acc[e] += a[u][e];
  }
  for (; r < chunk; r += RPL) {
    float a[VEC];
    load16<T>(base + static_cast<int64_t>(r) * D, a);
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] += a[e];
  }
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] += __shfl_xor(acc[e], off, kWave);
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
    int64_t summary_chunks, int64_t chunk_begin, int64_t nreq) {
  const int64_t bh = blockIdx.x / nreq;
  const int64_t c = chunk_begin + blockIdx.x % nreq;
  const T* __restrict__ base = k + (bh * seq_len + c * chunk) * D;
  const float fc = static_cast<float>(chunk);
  for (int d = threadIdx.x; d < D; d += kWave) {
    float a = 0.f;
    for (int r = 0; r < chunk; ++r) a += to_f32(base[static_cast<int64_t>(r) * D + d]);
    summary[(bh * summary_chunks + c) * D + d] = a / fc;
  }
}

// ---------------------------------------------------------------------------
// Chunk scores: score[c] = (q . summary[c]) * scale, fp32 (reference.py:54-55).
// Summary rows are fp32: a lane loads 4 columns; R chunks per wavefront.
// ---------------------------------------------------------------------------
template <typename T, int D, int R>
__global__ __launch_bounds__(64) void csa_score_vec_kernel(const T* __restrict__ q,
                                                           const float* __restrict__ summary,
                                                           float* __restrict__ scores,
                                                           int64_t C, int64_t blocks_per_head,
                                                           float scale) {
  constexpr int LPR = D / 4;
  constexpr int RPL = kWave / LPR;
  static_assert(R % RPL == 0, "R must be a multiple of rows per load");
  constexpr int U = R / RPL;
  const int lane = threadIdx.x;
  const int grp = lane / LPR;
  const int col = lane % LPR;
  const int64_t bh = blockIdx.x / blocks_per_head;
  const int64_t c0 = (blockIdx.x % blocks_per_head) * R;
  float qf[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) qf[e] = to_f32(q[bh * D + col * 4 + e]);
  const float* __restrict__ sb = summary + bh * C * D + col * 4;
  float sc[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t c = c0 + grp + RPL * u;
    float a[4] = {0.f, 0.f, 0.f, 0.f};
    if (c < C) load16<float>(sb + c * D, a);
    float d = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) d = fmaf(qf[e], a[e], d);
    sc[u] = d;
  }
#pragma unroll
  for (int off = LPR / 2; off >= 1; off >>= 1)
#pragma unroll
    for (int u = 0; u < U; ++u) sc[u] += __shfl_xor(sc[u], off, kWave);
  if (col == 0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t c = c0 + grp + RPL * u;
      if (c < C) scores[bh * C + c] = sc[u] * scale;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(64) void csa_score_generic_kernel(const T* __restrict__ q,
                                                               const float* __restrict__ summary,
                                                               float* __restrict__ scores, int64_t C,
                                                               int D, float scale) {
  const int64_t bh = blockIdx.x / C;
  const int64_t c = blockIdx.x % C;
  float d = 0.f;
  for (int j = threadIdx.x; j < D; j += kWave)
    d = fmaf(to_f32(q[bh * D + j]), summary[(bh * C + c) * D + j], d);
  d = wave_sum(d);
  if (threadIdx.x == 0) scores[bh * C + c] = d * scale;
}

// ---------------------------------------------------------------------------
// Top-k chunk selection (torch.topk in reference.py:56, with the declared
// tie-break: higher score first, equal scores by lower chunk id).
// One wavefront per (b,h):
//   * radix select (4 passes of 8 bits, LDS histograms) finds the k-th largest
//     order key T and how many keys equal to T are needed;
//   * keys > T are gathered (any order), then the needed keys == T in ascending
//     chunk order (ballot + prefix popcount);
//   * each winner's output position is its rank among the k winners.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__global__ __launch_bounds__(64) void csa_topk_kernel(const float* __restrict__ scores,
                                                      int32_t* __restrict__ out, int64_t C, int k) {
  extern __shared__ uint32_t lds[];
  uint32_t* hist = lds;                                      // 256
  uint32_t* skey = lds + 256;                                // k
  int32_t* sidx = reinterpret_cast<int32_t*>(skey + k);      // k
  __shared__ uint32_t s_count;
  const int lane = threadIdx.x;
  const int64_t bh = blockIdx.x;
  const float* __restrict__ sc = scores + bh * C;

  uint32_t prefix = 0, pmask = 0;
  uint32_t need = static_cast<uint32_t>(k);  // rank of the k-th key among the candidates
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
    for (int b = lane; b < 256; b += kWave) hist[b] = 0;
    __syncthreads();
    for (int64_t i = lane; i < C; i += kWave) {
      const uint32_t key = order_key(sc[i]);
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    const uint32_t h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2],
                   h3 = hist[4 * lane + 3];
    const uint32_t mine = h0 + h1 + h2 + h3;
    uint32_t incl = mine;  // sum over lanes >= this lane (higher digits)
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t t = __shfl_down(incl, off, kWave);
      if (lane + off < kWave) incl += t;
    }
    uint32_t cum = incl - mine;  // keys whose digit is above this lane's bins
    int found = -1;
    uint32_t rest = 0;
    const uint32_t hb[4] = {h3, h2, h1, h0};
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      if (found < 0 && cum < need && cum + hb[b] >= need) {
        found = 4 * lane + 3 - b;
        rest = need - cum;
      }
      cum += hb[b];
    }
    const unsigned long long bal = __ballot(found >= 0);
    // Exactly one lane finds the digit (the candidates always number >= need);
    // fall back to lane 0 / digit 0 rather than read an undefined lane.
    const int src = bal ? __ffsll(static_cast<long long>(bal)) - 1 : 0;
    const int digit = bal ? __shfl(found, src, kWave) : 0;
    need = bal ? static_cast<uint32_t>(__shfl(static_cast<int>(rest), src, kWave)) : need;
    need = need < 1u ? 1u : (need > static_cast<uint32_t>(k) ? static_cast<uint32_t>(k) : need);
    prefix |= static_cast<uint32_t>(digit) << shift;
    pmask |= 0xffu << shift;
    __syncthreads();
  }
  const uint32_t T = prefix;
  const int n_above = k - static_cast<int>(need);
  if (lane == 0) s_count = 0;
  __syncthreads();
  for (int64_t i = lane; i < C; i += kWave) {
    const uint32_t key = order_key(sc[i]);
    if (key > T) {
      const uint32_t pos = atomicAdd(&s_count, 1u);
      if (pos < static_cast<uint32_t>(k)) {
        skey[pos] = key;
        sidx[pos] = static_cast<int32_t>(i);
      }
    }
  }
  uint32_t taken = 0;
  for (int64_t base = 0; base < C && taken < need; base += kWave) {
    const int64_t i = base + lane;
    const bool eq = i < C && order_key(sc[i]) == T;
    const unsigned long long bal = __ballot(eq);
    const uint32_t before = static_cast<uint32_t>(__popcll(bal & ((1ull << lane) - 1ull)));
    if (eq && taken + before < need) {
      skey[n_above + taken + before] = T;
      sidx[n_above + taken + before] = static_cast<int32_t>(i);
    }
    taken += static_cast<uint32_t>(__popcll(bal));
  }
  __syncthreads();
  for (int j = lane; j < k; j += kWave) {
    const uint32_t kj = skey[j];
    const int32_t ij = sidx[j];
    int r = 0;
    for (int i = 0; i < k; ++i) {
      const uint32_t ki = skey[i];
      const int32_t ii = sidx[i];
      r += (ki > kj) || (ki == kj && ii < ij);
    }
    out[bh * k + r] = ij;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
constexpr int kMaxTopkSelect = 4096;  // LDS bound of csa_topk_kernel

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
    csa_attend_vec_kernel<T, IdxT, (DD / VEC <= kWave ? DD : VEC), 4><<<grid, kWave, 0, stream>>>( \
        qp, kp, vp, ip, part_ml, part_acc, S, top_k, chunk, cshift, tile, num_tiles, qscale);  \
    CSAHCA_LAUNCH_CHECK("csa_attend_vec_kernel");                                            \
    return CSAHCA_OK;                                                                        \
  }
  CSAHCA_ATTEND_VEC(64)
  CSAHCA_ATTEND_VEC(128)
  CSAHCA_ATTEND_VEC(256)
  CSAHCA_ATTEND_VEC(512)
#undef CSAHCA_ATTEND_VEC
  const int64_t J = ceil_div(D, kWave);
#define CSAHCA_ATTEND_GEN(JJ)                                                                  \
  if (J <= JJ) {                                                                               \
    csa_attend_generic_kernel<T, IdxT, JJ><<<grid, kWave, 0, stream>>>(                        \
        qp, kp, vp, ip, part_ml, part_acc, S, static_cast<int>(D), top_k, chunk, cshift, tile, \
        num_tiles, qscale);                                                                    \
    CSAHCA_LAUNCH_CHECK("csa_attend_generic_kernel");                                        \
    return CSAHCA_OK;                                                                          \
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
                    int64_t top_k, int64_t chunk, int64_t tile, const char* kernel_name,
                    void* workspace, size_t workspace_bytes, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(valid_dtype(dtype), "q, k_cache and v_cache must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(index_dtype == CSAHCA_I32 || index_dtype == CSAHCA_I64,
                 "chunk_indices must be int32 or int64");
  CSAHCA_REQUIRE(B >= 0 && H >= 0 && S >= 0 && D >= 0 && top_k >= 0, "negative dimension");
  CSAHCA_REQUIRE(chunk > 0, "chunk_size must be positive");
  CSAHCA_REQUIRE(tile > 0, "tile_size must be positive");
  CSAHCA_REQUIRE(D <= 1024, kernel_name);
  CSAHCA_REQUIRE(top_k * chunk <= INT_MAX, "top_k * chunk_size must fit in int32");
  CSAHCA_REQUIRE(chunk <= INT_MAX && top_k <= INT_MAX, "chunk_size and top_k must fit in int32");
  const int64_t bh = B * H;
  if (bh == 0 || D == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(q && k && v && out && (idx || top_k == 0), "null tensor pointer");
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
  // A null chunk list (top_k == 0) never dereferences idx: every slot range is empty.
  const void* idx_ok = idx ? idx : q;
  return dispatch_dtype(dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    int rc = index_dtype == CSAHCA_I32
                 ? launch_attend<T, int32_t>(q, k, v, idx_ok, part_ml, part_acc, bh, S, D,
                                             static_cast<int>(top_k), static_cast<int>(chunk), tl,
                                             static_cast<int>(tiles), stream)
                 : launch_attend<T, int64_t>(q, k, v, idx_ok, part_ml, part_acc, bh, S, D,
                                             static_cast<int>(top_k), static_cast<int>(chunk), tl,
                                             static_cast<int>(tiles), stream);
    if (rc != CSAHCA_OK) return rc;
    const int threads = static_cast<int>(std::min<int64_t>(256, ceil_div(D, kWave) * kWave));
    csa_merge_kernel<T><<<dim3(static_cast<uint32_t>(bh)), threads, 0, stream>>>(
        part_ml, part_acc, static_cast<T*>(out), static_cast<int>(D), static_cast<int>(tiles));
    CSAHCA_LAUNCH_CHECK("csa_merge_kernel");
    return CSAHCA_OK;
  });
}

}  // namespace
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

extern "C" int csahca_csa_chunk_summary(const void* k_cache, float* summary, int dtype,
                                        int64_t batch, int64_t heads, int64_t seq_len,
                                        int64_t head_dim, int64_t chunk_size,
                                        int64_t summary_chunks, int64_t chunk_begin,
                                        int64_t num_chunks, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(valid_dtype(dtype), "k_cache must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(batch >= 0 && heads >= 0 && seq_len >= 0 && head_dim >= 0, "negative dimension");
  CSAHCA_REQUIRE(chunk_size > 0 && chunk_size <= INT_MAX, "chunk_size must be positive");
  CSAHCA_REQUIRE(chunk_begin >= 0 && num_chunks >= 0, "chunk range must be non-negative");
  CSAHCA_REQUIRE((chunk_begin + num_chunks) * chunk_size <= seq_len,
                 "requested chunks extend past seq_len (only complete chunks have summaries)");
  CSAHCA_REQUIRE(summary_chunks >= chunk_begin + num_chunks, "summary has too few chunk rows");
  CSAHCA_REQUIRE(head_dim <= 1024, "head_dim > 1024 is not supported");
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
    csa_summary_vec_kernel<T, (DD / VEC <= kWave ? DD : VEC)><<<grid, kWave, 0, stream>>>(   \
        kp, summary, seq_len, static_cast<int>(chunk_size), summary_chunks, chunk_begin,     \
        num_chunks);                                                                         \
    CSAHCA_LAUNCH_CHECK("csa_summary_vec_kernel");                                         \
    return CSAHCA_OK;                                                                        \
  }
    CSAHCA_SUM_VEC(64)
    CSAHCA_SUM_VEC(128)
    CSAHCA_SUM_VEC(256)
    CSAHCA_SUM_VEC(512)
#undef CSAHCA_SUM_VEC
    csa_summary_generic_kernel<T><<<grid, kWave, 0, stream>>>(
        kp, summary, seq_len, static_cast<int>(head_dim), static_cast<int>(chunk_size),
        summary_chunks, chunk_begin, num_chunks);
    CSAHCA_LAUNCH_CHECK("csa_summary_generic_kernel");
    return CSAHCA_OK;
  });
}

extern "C" size_t csahca_csa_select_workspace_bytes(int64_t batch, int64_t heads,
                                                    int64_t num_chunks) {
  if (batch < 0 || heads < 0 || num_chunks < 0) return 0;
  return static_cast<size_t>(batch * heads * num_chunks) * sizeof(float);
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
  const int64_t bh = batch * heads;
  if (bh == 0 || k == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(q && summary && out_indices, "null tensor pointer");
  CSAHCA_REQUIRE(bh * num_chunks <= INT32_MAX, "too many chunks in one call");
  const size_t need = csahca_csa_select_workspace_bytes(batch, heads, num_chunks);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(CSAHCA_ERR_WORKSPACE, "workspace too small for csa select");
  float* scores = static_cast<float*>(workspace);
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  const float scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  const bool aligned = reinterpret_cast<uintptr_t>(summary) % 16 == 0;
  int rc = dispatch_dtype(dtype, [&](auto tag) -> int {
    using T = decltype(tag);
    const T* qp = static_cast<const T*>(q);
#define CSAHCA_SCORE_VEC(DD, RR)                                                           \
  if (aligned && head_dim == DD) {                                                         \
    const int64_t bph = ceil_div(num_chunks, RR);                                          \
    csa_score_vec_kernel<T, DD, RR><<<dim3(static_cast<uint32_t>(bh * bph)), kWave, 0,     \
                                      stream>>>(qp, summary, scores, num_chunks, bph, scale); \
    CSAHCA_LAUNCH_CHECK("csa_score_vec_kernel");                                         \
    return CSAHCA_OK;                                                                      \
  }
    CSAHCA_SCORE_VEC(64, 16)
    CSAHCA_SCORE_VEC(128, 16)
    CSAHCA_SCORE_VEC(256, 8)
#undef CSAHCA_SCORE_VEC
    csa_score_generic_kernel<T><<<dim3(static_cast<uint32_t>(bh * num_chunks)), kWave, 0, stream>>>(
        qp, summary, scores, num_chunks, static_cast<int>(head_dim), scale);
    CSAHCA_LAUNCH_CHECK("csa_score_generic_kernel");
    return CSAHCA_OK;
  });
  if (rc != CSAHCA_OK) return rc;
  const size_t lds = (256 + 2 * static_cast<size_t>(k)) * sizeof(uint32_t);
  csa_topk_kernel<<<dim3(static_cast<uint32_t>(bh)), kWave, lds, stream>>>(
      scores, out_indices, num_chunks, static_cast<int>(k));
  CSAHCA_LAUNCH_CHECK("csa_topk_kernel");
  return CSAHCA_OK;
}
