// csa_device.hpp -- wavefront-level building blocks of the CSA decode kernels.
#pragma once

#include "common.hpp"

namespace csahca {

// Order-preserving map fp32 -> uint32 (larger float -> larger key; +NaN above +inf).
__device__ __forceinline__ uint32_t order_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Number of set bits of a ballot below this lane (v_mbcnt_lo/hi).
__device__ __forceinline__ int lanes_below(unsigned long long bal) {
  return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0u)));
}

// Slot s -> token of chunk ids[s / chunk] (chunk_shift >= 0 when chunk is a
// power of two).  False when the chunk id is negative or the token is past
// seq_len (csrc/csa_attention.cu:176-185).
template <typename GetId>
__device__ __forceinline__ bool slot_token_of(GetId get_id, int s, int chunk, int chunk_shift,
                                              int64_t seq_len, int64_t& tok) {
  int cs, off;
  if (chunk_shift >= 0) {
    cs = s >> chunk_shift;
    off = s & (chunk - 1);
  } else {
    cs = s / chunk;
    off = s - cs * chunk;
  }
  const int64_t c = static_cast<int64_t>(get_id(cs));
  tok = c * chunk + off;
  return c >= 0 && tok < seq_len;
}

// ---------------------------------------------------------------------------
// Top-k over uint32 keys held in LDS, executed by ONE wavefront.
// Declared order: larger key first, equal keys by lower position first.
//   radix select (4 x 8-bit digits, LDS histogram) -> k-th key T and how many
//   keys equal to T are needed; gather keys > T, then the needed T keys in
//   ascending position (ballot + prefix popcount); rank the k winners.
// Scratch: hist[256], skey[k], sidx[k], counter[1].  Output: out[rank] = position.
// ---------------------------------------------------------------------------
template <typename Out>
__device__ void wave_topk_lds(const uint32_t* keys, int C, int k, uint32_t* hist, uint32_t* skey,
                              int32_t* sidx, uint32_t* counter, Out out) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t prefix = 0, pmask = 0;
  uint32_t need = static_cast<uint32_t>(k);
  for (int pass = 0; pass < 4; ++pass) {
    const int shift = 24 - 8 * pass;
#pragma unroll
    for (int b = 0; b < 4; ++b) hist[lane + kWave * b] = 0;
    wave_lds_sync();
    for (int i = lane; i < C; i += kWave) {
      const uint32_t key = keys[i];
      if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    wave_lds_sync();
    const uint32_t h0 = hist[4 * lane], h1 = hist[4 * lane + 1], h2 = hist[4 * lane + 2],
                   h3 = hist[4 * lane + 3];
    const uint32_t mine = h0 + h1 + h2 + h3;
    uint32_t incl = mine;  // keys whose digit lies in bins owned by lanes >= this lane
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t t = __shfl_down(incl, off, kWave);
      if (lane + off < kWave) incl += t;
    }
    uint32_t cum = incl - mine;
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
    const int src = bal ? __ffsll(static_cast<long long>(bal)) - 1 : 0;
    const int digit = bal ? __shfl(found, src, kWave) : 0;
    if (bal) need = static_cast<uint32_t>(__shfl(static_cast<int>(rest), src, kWave));
    need = need < 1u ? 1u : (need > static_cast<uint32_t>(k) ? static_cast<uint32_t>(k) : need);
    prefix |= static_cast<uint32_t>(digit) << shift;
    pmask |= 0xffu << shift;
    wave_lds_sync();
  }
  const uint32_t T = prefix;
  const uint32_t n_above = static_cast<uint32_t>(k) - need;
  if (lane == 0) *counter = 0;
  wave_lds_sync();
  for (int i = lane; i < C; i += kWave) {
    const uint32_t key = keys[i];
    if (key > T) {
      const uint32_t pos = atomicAdd(counter, 1u);
      if (pos < n_above) {
        skey[pos] = key;
        sidx[pos] = i;
      }
    }
  }
  uint32_t taken = 0;
  for (int base = 0; base < C && taken < need; base += kWave) {
    const int i = base + lane;
    const bool eq = i < C && keys[i] == T;
    const unsigned long long bal = __ballot(eq);
    const uint32_t before = static_cast<uint32_t>(lanes_below(bal));
    if (eq && taken + before < need) {
      skey[n_above + taken + before] = T;
      sidx[n_above + taken + before] = i;
    }
    taken += static_cast<uint32_t>(__popcll(bal));
  }
  wave_lds_sync();
  for (int j = lane; j < k; j += kWave) {
    const uint32_t kj = skey[j];
    const int32_t ij = sidx[j];
    int r = 0;
    for (int i = 0; i < k; ++i) {
      const uint32_t ki = skey[i];
      const int32_t ii = sidx[i];
      r += (ki > kj) || (ki == kj && ii < ij);
    }
    out(r, ij);
  }
  wave_lds_sync();
}

// LDS scratch of the register-path top-k: 64 candidate composites (u64) and
// one dummy slot that absorbs the stores of lanes without a candidate.
constexpr int kTopkScratchWords = 2 * (64 + 1);
constexpr int kCandBytes = kTopkScratchWords * 4;

// Compare-exchange at distance D keeping the larger value in the lower lane.
template <int D>
__device__ __forceinline__ uint32_t cx_desc(uint32_t x, int lane) {
  const uint32_t p = lane_xor<D>(x, lane);
  return (lane & D) ? (x < p ? x : p) : (x < p ? p : x);
}

template <int D>
__device__ __forceinline__ uint32_t merge_desc(uint32_t x, int lane) {
  x = cx_desc<D>(x, lane);
  if constexpr (D > 1) x = merge_desc<D / 2>(x, lane);
  return x;
}

// All-ones in lanes whose bit B is set.
template <int B>
__device__ __forceinline__ uint32_t lane_bit_mask(int lane) {
  return static_cast<uint32_t>(-((lane >> B) & 1));
}

// Sorts one value per lane across the wavefront, largest in lane 0: a bitonic
// network whose blocks of size S end descending where (lane & S) == 0 and
// ascending elsewhere.  Lanes of ascending blocks hold the complement (which
// reverses the order), so every compare-exchange keeps the larger value in
// the lower lane; the complement pattern is switched between stages.
__device__ __forceinline__ uint32_t wave_sort_desc(uint32_t x, int lane) {
  x ^= lane_bit_mask<1>(lane);
  x = merge_desc<1>(x, lane);
  x ^= lane_bit_mask<1>(lane) ^ lane_bit_mask<2>(lane);
  x = merge_desc<2>(x, lane);
  x ^= lane_bit_mask<2>(lane) ^ lane_bit_mask<3>(lane);
  x = merge_desc<4>(x, lane);
  x ^= lane_bit_mask<3>(lane) ^ lane_bit_mask<4>(lane);
  x = merge_desc<8>(x, lane);
  x ^= lane_bit_mask<4>(lane) ^ lane_bit_mask<5>(lane);
  x = merge_desc<16>(x, lane);
  x ^= lane_bit_mask<5>(lane);
  return merge_desc<32>(x, lane);
}

// The k-th largest (k <= 8) of one value per lane, in every lane: each block
// of 8 lanes is sorted descending (6 stages, as wave_sort_desc's first
// three merges but with every block descending), then three levels merge
// blocks 8, 16 and 32 lanes apart: lane i of a block takes the larger of its
// value and lane 7 - i of the partner block (a mirrored permute), which leaves
// the top 8 of both blocks as a bitonic sequence, and a 3-stage merge sorts
// it descending again.  18 stages against the full sort's 21; afterwards
// every block holds the wavefront's top 8 in descending order.
__device__ __forceinline__ uint32_t wave_top8_desc(uint32_t x, int lane) {
  x ^= lane_bit_mask<1>(lane);
  x = merge_desc<1>(x, lane);
  x ^= lane_bit_mask<1>(lane) ^ lane_bit_mask<2>(lane);
  x = merge_desc<2>(x, lane);
  x ^= lane_bit_mask<2>(lane);
  x = merge_desc<4>(x, lane);
  uint32_t p = dpp_mov<0x140>(x);  // row_mirror: lane ^ 15 (the block 8 lanes away, mirrored)
  x = x > p ? x : p;
  x = merge_desc<4>(x, lane);
  p = dpp_mov<0x141>(lane_xor<16>(x, lane));  // half_row_mirror after the row swap: lane ^ 16 ^ 7
  x = x > p ? x : p;
  x = merge_desc<4>(x, lane);
  p = dpp_mov<0x141>(lane_xor<32>(x, lane));  // lane ^ 32 ^ 7
  x = x > p ? x : p;
  return merge_desc<4>(x, lane);
}

// ---------------------------------------------------------------------------
// Top-k for k <= 64, executed by ONE wavefront.  On gfx950 every dependent
// hop between the vector and the scalar unit (a compare whose mask feeds a
// scalar op that feeds the next vector op) costs ~100 cycles and an LDS round
// trip ~120, so the steps avoid both:
//   1. each lane holds M keys in registers, row j of 64 positions rotated by
//      j (lane L holds position 64 j + ((L - j) mod 64)), and takes their
//      maximum.  The rotation puts the two natural shapes of a selection on
//      distinct lanes: chunks at a common stride of at least M, and any
//      contiguous run of at most 63 chunks; their maxima then sit in
//      different lanes and step 2 finds a tight threshold;
//   2. t = the k-th largest of the 64 lane maxima, from a network of lane
//      permutes (no LDS): the top-8 network for k <= 8, else the full
//      bitonic sort.  At least k keys are >= t and every key of the answer is
//      >= t;
//   3. keys >= t are compacted into LDS as unique composites
//      (key << 32 | ~position) in one pass: each lane counts its candidates,
//      one ballot per bit of the counts and mbcnt give every lane its first
//      slot (no scalar count carried from key to key);
//   4. with n <= 64 candidates, lane j ranks composite j by counting the
//      larger composites from broadcast reads (16 per batch, one LDS wait
//      each); composite order is exactly the declared order (larger key
//      first, equal keys by lower position).
// Returns false (nothing emitted) when more than 64 keys are >= t, or when
// t == 0 (fewer than k lanes hold a key, or keys equal to 0 decide the
// answer); the caller then runs wave_topk_lds.
// ---------------------------------------------------------------------------
template <int M, typename Out>
__device__ bool wave_topk_regs(const uint32_t* keys, int C, int k, uint32_t* scratch, Out out) {
  const int lane = threadIdx.x & (kWave - 1);
  unsigned long long* cand = reinterpret_cast<unsigned long long*>(scratch);
  uint32_t v[M];
#pragma unroll
  for (int j = 0; j < M; ++j) {
    // Clamped load + select rather than a branch per key (C >= 1).
    const int i = kWave * j + ((lane - j) & (kWave - 1));
    const uint32_t kv = keys[i < C ? i : C - 1];
    v[j] = i < C ? kv : 0u;
  }
  cand[lane] = 0ull;  // unused slots: below every composite (positions are < 2^31)
  uint32_t mx = 0;
#pragma unroll
  for (int j = 0; j < M; ++j) mx = v[j] > mx ? v[j] : mx;
  const uint32_t srt = k <= 8 ? wave_top8_desc(mx, lane) : wave_sort_desc(mx, lane);
  const uint32_t t = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(srt), k - 1));
  if (t == 0u) return false;
  wave_lds_sync();  // the clears above land before any compacted store
  // Positions past C hold key 0 < t, so no bound check is needed.
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < M; ++j) cnt += v[j] >= t ? 1 : 0;
  // This lane's first slot = the candidates of the lanes below it, bit by bit
  // of the counts (0 .. M); n = all candidates.
  int slot = 0, n = 0;
#pragma unroll
  for (int b = 0; (1 << b) <= M; ++b) {
    const unsigned long long bal = __ballot((cnt >> b) & 1);
    slot += lanes_below(bal) << b;
    n += __popcll(bal) << b;
  }
#pragma unroll
  for (int j = 0; j < M; ++j) {
    // Keys below t (and candidates past 64) store to the dummy slot.
    const bool take = v[j] >= t;
    const int sj = take && slot < kWave ? slot : kWave;
    const uint32_t pos = static_cast<uint32_t>(kWave * j + ((lane - j) & (kWave - 1)));
    cand[sj] = (static_cast<unsigned long long>(v[j]) << 32) | static_cast<uint32_t>(~pos);
    slot += take ? 1 : 0;
  }
  if (n > kWave) return false;
  wave_lds_sync();
  if (lane < n) {
    const unsigned long long cj = cand[lane];
    int r = 0;
    for (int b = 0; b < n; b += 16) {  // slots [n, 64) hold 0
      ulonglong2 c2[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) c2[i] = *reinterpret_cast<const ulonglong2*>(cand + b + 2 * i);
#pragma unroll
      for (int i = 0; i < 8; ++i) r += (c2[i].x > cj) + (c2[i].y > cj);
    }
    if (r < k) out(r, static_cast<int32_t>(~static_cast<uint32_t>(cj)));
  }
  wave_lds_sync();
  return true;
}

// Position of the largest key of keys[0, C) (1 <= C <= 64 * M), larger key
// first and equal keys by lower position: the first slot of every top-k
// above.  Each lane reads its M keys in one batch (position 64 j + lane;
// positions past C read as key 0 at a position above every real one, so they
// never win a tie), keeps its best, and a butterfly of lane exchanges (DPP and
// row swaps, no LDS) takes the best of all lanes in the same order: every
// lane ends with the answer.  The whole wavefront must be active.
template <int M>
__device__ __forceinline__ int32_t wave_top1(const uint32_t* keys, int C) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t v[M];
#pragma unroll
  for (int j = 0; j < M; ++j) {
    const int i = kWave * j + lane;
    const uint32_t kv = keys[i < C ? i : C - 1];
    v[j] = i < C ? kv : 0u;
  }
  uint32_t bk = v[0], bp = static_cast<uint32_t>(lane);
#pragma unroll
  for (int j = 1; j < M; ++j) {  // positions rise with j: a later equal key loses
    const bool take = v[j] > bk;
    bk = take ? v[j] : bk;
    bp = take ? static_cast<uint32_t>(kWave * j + lane) : bp;
  }
  // One 64-bit compare per exchange: key << 32 | ~position orders exactly so.
  unsigned long long c = (static_cast<unsigned long long>(bk) << 32) | static_cast<uint32_t>(~bp);
  auto step = [&](uint32_t hi, uint32_t lo) {
    const unsigned long long o = (static_cast<unsigned long long>(hi) << 32) | lo;
    c = o > c ? o : c;
  };
  auto hi = [&] { return static_cast<uint32_t>(c >> 32); };
  auto lo = [&] { return static_cast<uint32_t>(c); };
  step(lane_xor<1>(hi(), lane), lane_xor<1>(lo(), lane));
  step(lane_xor<2>(hi(), lane), lane_xor<2>(lo(), lane));
  step(lane_xor<4>(hi(), lane), lane_xor<4>(lo(), lane));
  step(lane_xor<8>(hi(), lane), lane_xor<8>(lo(), lane));
  step(lane_xor<16>(hi(), lane), lane_xor<16>(lo(), lane));
  step(lane_xor<32>(hi(), lane), lane_xor<32>(lo(), lane));
  return static_cast<int32_t>(~static_cast<uint32_t>(c));
}

// Register-path size for a selection: keys per lane M (C <= 64 * M), or 0 for
// the LDS radix path only.  Kernels take M as a template parameter so each
// instantiation carries exactly one register path.
inline int topk_regs_for(int64_t C, int64_t k) {
  if (k > kWave) return 0;
  if (C <= 512) return 8;
  if (C <= 2048) return 32;
  return 0;
}

// Top-k with the declared order: the register path when M > 0 (falling back
// when too many keys tie around its threshold), else the LDS radix select.
template <int M, typename Out>
__device__ __forceinline__ void wave_topk(const uint32_t* keys, int C, int k, uint32_t* scratch,
                                          uint32_t* hist, uint32_t* skey, int32_t* sidx,
                                          uint32_t* counter, Out out) {
  if constexpr (M > 0) {
    if (k <= kWave && wave_topk_regs<M>(keys, C, k, scratch, out)) return;
  }
  wave_topk_lds(keys, C, k, hist, skey, sidx, counter, out);
}

// ---------------------------------------------------------------------------
// Online-softmax state of one wavefront over rows of a [*, D] K/V pair, with
// the row split of csa_attend: each lane owns VEC = 16/sizeof(T) columns, a
// wavefront-wide 16-byte load covers RPL = 64 / (D / VEC) rows.  Scores are in
// the base-2 domain (q pre-scaled by log2(e)/sqrt(D)).
// ---------------------------------------------------------------------------
template <typename T, int D>
struct AttendLayout {
  static constexpr int VEC = Vec16<T>::N;
  static constexpr int LPR = D / VEC;
  static constexpr int RPL = kWave / LPR;
  static_assert(LPR >= 1 && LPR <= kWave && (LPR & (LPR - 1)) == 0, "bad row split");
};

// Column sums of `chunk` consecutive [*, D] rows by one wavefront in the
// AttendLayout split: lane (grp, col) adds rows grp, grp + RPL, ... of its VEC
// columns at `base` (row 0, column col * VEC), U rows per batch of loads, then
// the row groups are folded by a butterfly, so every lane ends with the sums
// of its columns.  The chunk-summary kernel (U = 16: a 64-row chunk in one
// batch) and the fused decode step (U = 4, in the few registers it has left)
// both build summaries through this one function; a lane adds its rows in row
// order whatever U is, so their rows agree bit for bit.
template <typename T, int D, int U = 4>
__device__ __forceinline__ void wave_chunk_colsum(const T* __restrict__ base, int chunk, int grp, float* acc) {
  using L = AttendLayout<T, D>;
  constexpr int VEC = L::VEC, LPR = L::LPR, RPL = L::RPL;
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  int r = grp;
  for (; r + (U - 1) * RPL < chunk; r += U * RPL) {
    float a[U][VEC];
#pragma unroll
    for (int u = 0; u < U; ++u) load16<T>(base + static_cast<int64_t>(r + u * RPL) * D, a[u]);
#pragma unroll
    for (int u = 0; u < U; ++u)
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
    for (int e = 0; e < VEC; ++e) acc[e] += xor_lanes(acc[e], off);
}

template <typename T, int D>
struct WaveSoftmax {
  static constexpr int VEC = AttendLayout<T, D>::VEC;
  float m, l;
  float acc[VEC];
  __device__ __forceinline__ void init() {
    m = -INFINITY;
    l = 0.f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.f;
  }
};

// K and V rows of one batch of a lane (rows base + grp + RPL*u, u < U):
// issued by attend_issue, consumed by attend_consume.
template <int U>
struct AttendRows {
  uint4 rk[U], rv[U];
  bool ok[U];
};

// Token lookup and the row loads of rows base + grp + RPL*u (u < U) of the
// slot range [.., s1): tok_of(s, tok) maps a slot to a token (false = skip).
// kb/vb point at this lane's columns of row 0 of the (b,h) cache.  Every row
// load is unconditional (a skipped slot reads row 0 and is zeroed when
// consumed).
template <typename T, int D, int U, typename TokOf>
__device__ __forceinline__ void attend_issue(AttendRows<U>& r, const T* __restrict__ kb, const T* __restrict__ vb,
                                             int base, int s1, int grp, TokOf tok_of) {
  constexpr int RPL = AttendLayout<T, D>::RPL;
  // Tokens first (chunk ids may come from global memory), then every row:
  // the empty asm takes all token positions, so no row load is scheduled
  // before the last id is known -- an id wait after a row load would, with
  // in-order wait counts, also wait for that row.
  int64_t toks[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    // Slots past s1 look up slot s1 - 1 (valid whenever this block runs) and
    // are dropped afterwards: the id lookup stays outside any branch.
    const int s = base + grp + RPL * u;
    int64_t tok = 0;
    const bool found = tok_of(s < s1 ? s : s1 - 1, tok);
    r.ok[u] = s < s1 && found;
    toks[u] = r.ok[u] ? tok : 0;
  }
  if constexpr (U == 4) {
    asm volatile("" : "+v"(toks[0]), "+v"(toks[1]), "+v"(toks[2]), "+v"(toks[3]));
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) asm volatile("" : "+v"(toks[u]));
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    r.rk[u] = load_global_u4(kb + toks[u] * D);
    r.rv[u] = load_global_u4(vb + toks[u] * D);
  }
}

// Scale this lane's 16 bytes of q by qscale (fp32).
template <typename T, int D>
__device__ __forceinline__ void attend_q(const uint4& q16, float qscale, float* qf) {
  widen16<T>(q16, qf);
#pragma unroll
  for (int e = 0; e < AttendLayout<T, D>::VEC; ++e) qf[e] *= qscale;
}

// Online-softmax update of st with one issued batch of rows.
template <typename T, int D, int U>
__device__ __forceinline__ void attend_consume(WaveSoftmax<T, D>& st, const AttendRows<U>& r, const float* qf) {
  using L = AttendLayout<T, D>;
  constexpr int VEC = L::VEC, LPR = L::LPR;
  float kr[U][VEC], vr[U][VEC];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint4 z = make_uint4(0u, 0u, 0u, 0u);
    widen16<T>(r.ok[u] ? r.rk[u] : z, kr[u]);
    widen16<T>(r.ok[u] ? r.rv[u] : z, vr[u]);
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
    for (int u = 0; u < U; ++u) sc[u] += xor_lanes(sc[u], off);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    sc[u] = r.ok[u] ? sc[u] : -INFINITY;
    mx = fmaxf(mx, sc[u]);
  }
#pragma unroll
  for (int off = LPR; off < kWave; off <<= 1) mx = fmaxf(mx, xor_lanes(mx, off));
  const float m_new = fmaxf(st.m, mx);
  if (m_new == -INFINITY) return;  // wavefront-uniform: nothing valid yet
  const float alpha = fast_exp2(st.m - m_new);
  st.l *= alpha;
#pragma unroll
  for (int e = 0; e < VEC; ++e) st.acc[e] *= alpha;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const float p = fast_exp2(sc[u] - m_new);
    st.l += p;
#pragma unroll
    for (int e = 0; e < VEC; ++e) st.acc[e] = fmaf(p, vr[u][e], st.acc[e]);
  }
  st.m = m_new;
}

// One batch issued and consumed: q (scaled here by qscale, qp at this lane's
// 16 bytes) is loaded after the rows -- the newest load, so one wait covers
// the batch and no hoisted use of q can make the rows wait -- so the 2U + 1
// loads of a lane are one batch in flight.
template <typename T, int D, int U, typename TokOf>
__device__ __forceinline__ void attend_block(WaveSoftmax<T, D>& st, const T* qp, float qscale,
                                             const T* __restrict__ kb, const T* __restrict__ vb,
                                             int base, int s1, int grp, TokOf tok_of) {
  AttendRows<U> r;
  attend_issue<T, D, U>(r, kb, vb, base, s1, grp, tok_of);
  float qf[AttendLayout<T, D>::VEC];
  attend_q<T, D>(load_global_u4(qp), qscale, qf);
  attend_consume<T, D, U>(st, r, qf);
}

// Several batches (base, base + stride, ... below s1), double-buffered: the
// rows of batch i + 1 are requested before batch i is consumed, so a lane
// keeps two batches in flight instead of waiting a memory round trip per
// batch.  Every load is unconditional (a load under a branch makes the
// compiler wait for every outstanding load at the join), and the last batch
// is consumed in a tail of its own.  q is loaded first.
template <typename T, int D, int U, typename TokOf>
__device__ __forceinline__ void attend_pipelined_from(WaveSoftmax<T, D>& st, AttendRows<U>& ra, const uint4& q16,
                                                      float qscale, const T* __restrict__ kb,
                                                      const T* __restrict__ vb, int base, int stride, int s1,
                                                      int grp, TokOf tok_of);

template <typename T, int D, int U, typename TokOf>
__device__ __forceinline__ void attend_pipelined(WaveSoftmax<T, D>& st, const T* qp, float qscale,
                                                 const T* __restrict__ kb, const T* __restrict__ vb, int base,
                                                 int stride, int s1, int grp, TokOf tok_of) {
  if (base >= s1) return;
  const uint4 q16 = load_global_u4(qp);
  AttendRows<U> ra;
  attend_issue<T, D, U>(ra, kb, vb, base, s1, grp, tok_of);
  attend_pipelined_from<T, D, U>(st, ra, q16, qscale, kb, vb, base, stride, s1, grp, tok_of);
}

// The same walk, its first batch (rows `base`..) and q already requested by
// the caller into ra and q16.
template <typename T, int D, int U, typename TokOf>
__device__ __forceinline__ void attend_pipelined_from(WaveSoftmax<T, D>& st, AttendRows<U>& ra, const uint4& q16,
                                                      float qscale, const T* __restrict__ kb,
                                                      const T* __restrict__ vb, int base, int stride, int s1,
                                                      int grp, TokOf tok_of) {
  // Two buffers in turn (no copy between them: a copy lets the compiler load
  // the next batch into the registers of the one still in flight, which makes
  // every load wait for its predecessor).  The last batch is consumed in a
  // tail of its own, so nothing is left in flight after the walk; base is
  // made wavefront-uniform so the tests are scalar branches.
  AttendRows<U> rb;
  float qf[AttendLayout<T, D>::VEC];
  attend_q<T, D>(q16, qscale, qf);
  base = __builtin_amdgcn_readfirstlane(base);
  for (;;) {
    if (base + stride >= s1) {
      attend_consume<T, D, U>(st, ra, qf);
      break;
    }
    attend_issue<T, D, U>(rb, kb, vb, base + stride, s1, grp, tok_of);
    attend_consume<T, D, U>(st, ra, qf);
    base += stride;
    if (base + stride >= s1) {
      attend_consume<T, D, U>(st, rb, qf);
      break;
    }
    attend_issue<T, D, U>(ra, kb, vb, base + stride, s1, grp, tok_of);
    attend_consume<T, D, U>(st, rb, qf);
    base += stride;
  }
}

// Transposed fold of the row groups (RPL groups of LPR lanes): each step at
// distance OFF (LPR, 2 LPR, ..., 32: the pairing of a butterfly over the
// groups, so every column sum has that butterfly's bits) halves the acc
// values a lane holds while it holds more than one.  A lane ends with kFoldKeep column sums, of columns
// col * VEC + base .. + kFoldKeep - 1; l is summed over the groups in every lane.
template <int M, int OFF>
__device__ __forceinline__ void fold_groups_t(float* v, int lane, int& base) {
  if constexpr (OFF < kWave) {
    if constexpr (M > 1) {
      constexpr int H = M / 2;
      // Bit-mask selects keep every array access at a constant index.
      const uint32_t up = (lane & OFF) ? 0xffffffffu : 0u;
#pragma unroll
      for (int i = 0; i < H; ++i) {
        const uint32_t lo = __float_as_uint(v[i]), hi = __float_as_uint(v[i + H]);
        const float send = __uint_as_float((lo & up) | (hi & ~up));
        const float keep = __uint_as_float((hi & up) | (lo & ~up));
        v[i] = keep + xor_lanes(send, OFF);
      }
      base += (lane & OFF) ? H : 0;
      fold_groups_t<H, OFF * 2>(v, lane, base);
    } else {
      v[0] += xor_lanes(v[0], OFF);
      fold_groups_t<1, OFF * 2>(v, lane, base);
    }
  }
}

template <typename T, int D>
struct FoldShare {
  static constexpr int VEC = AttendLayout<T, D>::VEC;
  static constexpr int RPL = AttendLayout<T, D>::RPL;
  static constexpr int kKeep = VEC / RPL > 0 ? VEC / RPL : 1;
};

// Returns the first column (within the lane's VEC) of its kKeep sums, which
// are left in st.acc[0 .. kKeep).
template <typename T, int D>
__device__ __forceinline__ int fold_row_groups_share(WaveSoftmax<T, D>& st) {
  using L = AttendLayout<T, D>;
  const int lane = static_cast<int>(__lane_id());
#pragma unroll
  for (int off = L::LPR; off < kWave; off <<= 1) st.l += xor_lanes(st.l, off);
  int base = 0;
  fold_groups_t<L::VEC, L::LPR>(st.acc, lane, base);
  return base;
}

}  // namespace csahca
