// csa_step.hip -- one-launch CSA decode step for gfx950:
//   chunk scores from cached fp32 summaries -> top-k chunk selection ->
//   split-KV sparse attention over the selected tokens -> partial merge.
//
// Each (b,h) head is served by P workgroups of 4 wavefronts:
//   A. workgroup p scores summary rows [Cs*p/P, Cs*(p+1)/P) of the head's Cs
//      rows and publishes the order keys (fp32 score -> monotone uint32) of
//      those below the chunk count C (C = Cs unless the count is read from
//      device memory, which lets a captured graph follow a growing cache);
//   B. every workgroup gathers the head's C keys into LDS and wavefront 0 runs
//      the top-k (same keys, deterministic algorithm: identical everywhere);
//      selection slots beyond C hold chunk -1 (skipped);
//   C. workgroup p attends the selected-token slots [T*p/P, T*(p+1)/P) (T = k *
//      chunk) -- chunk ids from LDS, K/V rows by 16-byte lane loads -- and folds
//      its 4 wavefronts' online-softmax states in LDS;
//   D. every workgroup publishes its partial (m, l, acc[D]); workgroup 0 of the
//      head gathers the P partials and merges them (log-sum-exp) into the
//      output.
// With P == 1 a workgroup owns its head and nothing crosses workgroups; the
// wide instantiation (8 wavefronts, P == 1) serves grids of about one head
// per CU with large selections.
//
// Cross-workgroup exchange without cache maintenance: on gfx950 an agent-scope
// fence writes back / invalidates the whole L2 of an XCD, which at hundreds of
// workgroups costs tens of microseconds.  Instead every exchanged 32-bit value
// travels in a 64-bit word (tag << 32 | value) written and read with
// device-scope atomic stores/loads, which are coherent across XCDs on their
// own.  The tag is this launch's number for the head (epoch[h] + 1, read at
// entry; the merging workgroup publishes it as the new epoch when done), so a
// reader accepts a word only once it belongs to the current launch and needs no
// separate ordering.  Every wait is bounded.  On time-out a sticky status bit
// is set, the head's output is NaN and its epoch becomes kPoisonEpoch: a
// partner that had not started could otherwise publish words a later launch
// would take for its own, so every later launch on a poisoned head skips its
// waits and writes NaN, until the workspace is zero-filled again.
// The workspace must be zero before the first launch and whenever the problem
// shape (B*H, chunks, head_dim, top_k, chunk) changes.
#include "csa_device.hpp"
#include "hca_device.hpp"

#include <algorithm>
#include <climits>
#include <cstdlib>
#include <mutex>
#include <type_traits>
#include <vector>

namespace csahca {

int csa_select_launch(const void* q, const float* summary, int32_t* out_indices, int dtype,
                      int64_t bh, int64_t C, int64_t D, int64_t k, uint32_t* keys,
                      hipStream_t stream);
int hca_merge_launch(int dtype, void* workspace, const void* blend_src, double blend_weight, void* out,
                     int64_t bh, int64_t C, int D, hipStream_t stream);
size_t hca_workspace_means_offset(int64_t n_scores);

namespace {

// Phase timeline (a diagnostic build of its own, with -DCSAHCA_STEP_TIMELINE:
// libcsahca_timeline.so, read by csahca_amd/timeline.py).  Thread 0 of each
// workgroup records the device wall clock (100 MHz) at the phase boundaries
// of the step: 0 entry, 1 phase A done (keys published), 2 keys gathered,
// 3 top-k done, 4 attention done, 5 partial published, 6 output written (the
// merging workgroup, or every workgroup when P = 1).  The product build
// compiles none of it.
#ifdef CSAHCA_STEP_TIMELINE
constexpr int kTimelineBlocks = 4096;
constexpr int kTimelineStamps = 8;
__device__ uint64_t g_timeline[kTimelineBlocks][kTimelineStamps];
#define CSAHCA_STAMP(i)                                                                   \
  do {                                                                                    \
    if (threadIdx.x == 0 && block < kTimelineBlocks) g_timeline[block][(i)] = wall_clock64(); \
  } while (0)
#else
#define CSAHCA_STAMP(i) \
  do {                  \
  } while (0)
#endif

constexpr int kStepWaves = 4;
constexpr int kStepThreads = kStepWaves * kWave;
constexpr int kStepMaxP = 64;
constexpr int kStepMaxK = 1024;
constexpr int kStepScoreUnroll = 8;   // summary rows per lane per batch of loads
constexpr int kStepAttendUnroll = 4;  // K/V row loads per lane per batch
constexpr int kRegMergeP = 8;         // partials per head merged from registers
constexpr size_t kStepLds = 64 * 1024;
constexpr uint32_t kSpinLimit = 1u << 20;  // polls per bounded wait (each with a short sleep)

struct StepParams {
  const void* q;
  const float* summary;
  const void* kcache;
  const void* vcache;
  void* out;
  int32_t* idx_out;
  uint32_t* status;
  uint32_t* epoch;     // [BH]
  uint64_t* keys;      // head h's tagged keys at h * key_stride
  uint64_t* part;      // head h's tagged partials (m, l, acc[D]) at h * part_stride + p * (D + 2)
  int64_t key_stride;
  int64_t part_stride;
  int64_t S;
  int64_t C;            // chunks in play (when c_dev is null)
  int64_t Cs;           // summary / key rows per head (C <= Cs)
  const int32_t* c_dev;  // chunks in play, read on the device (clamped to [0, Cs]); may be null
  const int64_t* pos_dev;  // position of the token just appended, or null: chunks in play are
                           // min((pos + 1) / chunk, Cs) and the summary row of the chunk the token
                           // completes is built first (into summary_out)
  float* summary_out;
  int chunk;
  int chunk_shift;
  int topk;
  int P;
  uint32_t colo_bh;  // nonzero: block b serves head b % colo_bh, its workgroup b / colo_bh (a head's
                     // workgroups on one XCD when colo_bh is a multiple of 8); zero: head b / P
  float score_scale;
  float qscale;
  uint32_t spin_limit;  // polls before a wait gives up (kSpinLimit; smaller only under the test switch)
  int32_t mute_p;       // test switch: workgroup mute_p of head 0 publishes nothing (-1: none)
};

// Wait (bounded) until *p carries `tag`; returns its value bits.  On time-out
// the sticky status bit is set and `bad` is raised: the caller poisons what it
// computes from the word (the head's output becomes NaN and the head is
// poisoned), so a lost partner never yields a plausible-looking result.
__device__ __forceinline__ uint32_t wait_tagged(const uint64_t* p, uint64_t w, uint32_t tag, uint32_t* status,
                                                uint32_t spin_limit, bool& bad) {
  uint32_t it = 0;
  while (static_cast<uint32_t>(w >> 32) != tag) {
    __builtin_amdgcn_s_sleep(1);
    w = get_raw(p);
    if (++it > spin_limit) {
      __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bad = true;
      break;
    }
  }
  return static_cast<uint32_t>(w);
}

// Wait (bounded) until every valid word of a batch carries `tag`, re-reading
// the whole batch each round: one round trip per round, whatever the number of
// words that were not ready when the batch was first read (waiting on them one
// at a time costs a round trip per word).  valid(j) tells the words of the
// batch that exist (a prefix); addr(j) is the address of word j.  On time-out
// the sticky status bit is set and `bad` raised.
template <int N, typename Addr, typename Valid>
__device__ __forceinline__ void wait_tagged_batch(Addr addr, Valid valid, uint64_t (&w)[N], uint32_t tag,
                                                  uint32_t* status, uint32_t spin_limit, bool& bad) {
  for (uint32_t it = 0;; ++it) {
    bool ready = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ready = ready && (!valid(j) || static_cast<uint32_t>(w[j] >> 32) == tag);
    if (ready) return;
    if (it >= spin_limit) {
      __hip_atomic_fetch_or(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      bad = true;
      return;
    }
    __builtin_amdgcn_s_sleep(1);
    // (word 0 exists whenever any does: the others re-read it, unconditionally)
#pragma unroll
    for (int j = 0; j < N; ++j) w[j] = get_raw(addr(valid(j) ? j : 0));
  }
}

// PIPE: walk several batches of rows double-buffered (an instantiation of its
// own, so the batch-by-batch kernel keeps its code).  W: wavefronts per
// workgroup (the wide instantiation serves a head from one workgroup of 8).
// MERGE: which merge of the P partials the instantiation holds -- kMergeRegs
// (P <= kRegMergeP, the host guarantees it), kMergeLds (P > kRegMergeP) or
// kMergeBoth (chosen by P at run time).  Leaving the other merge out keeps the
// code of the latency-bound kernel smaller: without the LDS merge the B1 H8
// S32768 top-8 step took 9.68 against 9.78 us (512 steps, same box).
constexpr int kMergeRegs = 0, kMergeLds = 1, kMergeBoth = 2;
template <typename T, int D, int TOPK_M, bool POS, bool PIPE = false, int W = kStepWaves, int MERGE = kMergeBoth>
__device__ __forceinline__ void csa_step_body(StepParams a, uint32_t block) {
  constexpr int NT = W * kWave;
  using L = AttendLayout<T, D>;
  constexpr int VEC = L::VEC, LPR = L::LPR, RPL = L::RPL;
  constexpr int SLPR = D / 4, SRPL = kWave / SLPR;  // fp32 summary rows
  constexpr int U = kStepAttendUnroll;
  constexpr int B8 = 8;                              // tagged key loads issued per batch
  constexpr int kGather = 8;                         // tagged partial loads per thread per batch

  // LDS: keys[max(Cs, P*(D+2))] (the head's keys, later the gathered
  //      partials; first, so that its address needs only preloaded arguments)
  //      | top-k scratch (16-byte aligned) | hist[256] | skey[k] | sidx[k] |
  //      sel[k] | count | comb
  extern __shared__ uint64_t smem64[];
  uint32_t* keys_l = reinterpret_cast<uint32_t*>(smem64);
  const int64_t keys_words = max<int64_t>(a.Cs, a.P > 1 ? int64_t{a.P} * (D + 2) : 0);
  uint32_t* tk_scratch = keys_l + ((keys_words + 3) & ~int64_t{3});
  uint32_t* hist = tk_scratch + kTopkScratchWords;
  uint32_t* skey = hist + 256;
  int32_t* sidx = reinterpret_cast<int32_t*>(skey + a.topk);
  int32_t* sel = sidx + a.topk;
  uint32_t* lcount = reinterpret_cast<uint32_t*>(sel + a.topk);
  float* comb = reinterpret_cast<float*>(lcount + 1);

  const int tid = threadIdx.x;
  const int wave = tid / kWave;
  const int lane = tid % kWave;
  const int P = a.P;
  const uint32_t cb = a.colo_bh;
  const int64_t h = cb ? block % cb : block / P;
  const int p = static_cast<int>(cb ? block / cb : block % P);
  const int64_t Cs = a.Cs;
  // Loads that depend on nothing are issued together, unconditionally, and
  // consumed only after the summary rows are requested, so phase A costs one
  // memory round trip: this launch's tag for the head (epoch + 1; every head
  // has an epoch word, read even when P = 1), the device count or position,
  // q in the summary lane layout, and the summary rows.  (They need only the
  // preloaded arguments and the block index.)
  const uint32_t epoch = __hip_atomic_load(&a.epoch[h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // Chunks in play: the host's count, or the device's, or the count implied
  // by the device position of the token just appended (POS: the position
  // mode, a separate instantiation so that the count modes compile without
  // it).  The device count and the position are requested here, with an
  // unconditional load (the epoch word stands in for an absent count), and
  // applied in phase A where the keys are published, after its row loads.
  int64_t C = Cs;  // the count modes set it in phase A (count_from_device)
  const bool c_on_dev = !POS && a.c_dev != nullptr;
  int32_t c_raw = 0;
  if constexpr (!POS)
    c_raw = load_global_raw<int32_t>(c_on_dev ? a.c_dev : reinterpret_cast<const int32_t*>(a.epoch + h));
  auto count_from_device = [&]() {
    int32_t v = c_raw;
    asm volatile("" : "+v"(v));  // consumed only here, after the row loads
    C = c_on_dev ? min<int64_t>(max<int32_t>(v, 0), Cs) : a.C;
  };
  int64_t pos_raw = 0;
  if constexpr (POS) pos_raw = load_global_raw<int64_t>(a.pos_dev);
  const T* __restrict__ q = static_cast<const T*>(a.q) + h * D;
  CSAHCA_STAMP(0);

  // ---- A: order keys of this workgroup's chunk range ----------------------
  {
    const int grp = lane / SLPR, col = lane % SLPR;
    const float* __restrict__ sb = a.summary + h * Cs * D + col * 4;
    // This workgroup's rows: 32-bit division whenever Cs * P fits (every
    // practical shape); a 64-bit division is a long scalar sequence on the
    // critical path of the step.
    int64_t c0, c1;
    if (Cs * P <= static_cast<int64_t>(UINT32_MAX)) {
      const uint32_t cs = static_cast<uint32_t>(Cs), up = static_cast<uint32_t>(P);
      c0 = cs * static_cast<uint32_t>(p) / up;
      c1 = cs * static_cast<uint32_t>(p + 1) / up;
    } else {
      c0 = Cs * p / P;
      c1 = Cs * (p + 1) / P;
    }
    constexpr int US = kStepScoreUnroll;
    constexpr int64_t kScoreStride = W * SRPL * US;
    // Rows blk + wave*SRPL*US + grp + SRPL*u (u < US); rows past the range
    // re-read row c0 (their scores are dropped).
    auto issue_rows = [&](int64_t blk, uint4 (&rs)[US]) {
      const int64_t base = blk + wave * SRPL * US;
#pragma unroll
      for (int u = 0; u < US; ++u) {
        const int64_t c = base + grp + SRPL * u;
        rs[u] = load_global_u4(sb + (c < c1 ? c : c0) * D);
      }
    };
    // q[col*4 .. col*4+3] in the summary lane layout.
    auto load_q4 = [&]() -> uint4 {
      if constexpr (sizeof(T) == 4) {
        return load_global_u4(q + col * 4);
      } else {
        const uint2 t2 = load_global_u2(q + col * 4);
        return make_uint4(t2.x, t2.y, 0u, 0u);
      }
    };
    auto score_rows = [&](int64_t blk, uint4 (&rs)[US], const uint4& q4) {
      const int64_t base = blk + wave * SRPL * US;
      // The epoch is consumed only here: the empty asm keeps the compiler from
      // hoisting its use above the row loads.
      uint32_t ep = epoch;
      asm volatile("" : "+v"(ep));
      uint64_t* kg = a.keys + h * a.key_stride;
      // Test switch only (the host sets mute_p = -1 otherwise): this workgroup
      // publishes no key and no partial, so its partners' bounded waits expire.
      const bool mute = h == 0 && p == a.mute_p;
      if constexpr (!POS) count_from_device();
      if constexpr (POS) {
        // The token at pos was just appended: n = pos + 1 tokens, C complete
        // chunks.  If it completes chunk C - 1 and this block of rows holds
        // that row, wavefront 0 builds the row first -- through the summary
        // kernel's own column-sum routine, so the bits are the summary
        // kernel's -- and the block's rows are loaded again (once every
        // `chunk` steps, in one workgroup per head).
        int64_t n = pos_raw;
        asm volatile("" : "+v"(n));  // consumed only here, after the loads above
        n += 1;
        const int64_t nc = n <= 0 ? 0 : (a.chunk_shift >= 0 ? n >> a.chunk_shift : n / a.chunk);
        C = min<int64_t>(nc, Cs);
        const int64_t cn = C - 1;
        const bool build = n > 0 && nc * a.chunk == n && nc <= Cs && n <= a.S;
        if (build && cn >= blk && cn < blk + W * SRPL * US && cn < c1) {
          if (wave == 0) {
            const int g2 = lane / LPR, c2 = lane % LPR;
            const T* kb0 = static_cast<const T*>(a.kcache) + (h * a.S + cn * a.chunk) * D + c2 * VEC;
            float acc[VEC];
            wave_chunk_colsum<T, D>(kb0, a.chunk, g2, acc);
            if (g2 == 0) {
              float* dst = a.summary_out + (h * Cs + cn) * D + c2 * VEC;
              const float fc = static_cast<float>(a.chunk);
#pragma unroll
              for (int e = 0; e < VEC; ++e) dst[e] = acc[e] / fc;
            }
            __threadfence();
          }
          __syncthreads();
#pragma unroll
          for (int u = 0; u < US; ++u) {
            const int64_t c = base + grp + SRPL * u;
            rs[u] = load_global_u4(sb + (c < c1 ? c : c0) * D);
          }
        }
      }
      float qf[8];
      widen16<T>(q4, qf);
      float sc[US];
#pragma unroll
      for (int u = 0; u < US; ++u) {
        float r4[4];
        widen16<float>(rs[u], r4);
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) d = fmaf(qf[e], r4[e], d);
        sc[u] = d;
      }
      // Row sums over the SLPR lanes of each row, transposed: lane col ends
      // with row u = col / (SLPR / US), and one lane per row publishes its key
      // (a wavefront's 16 B-row keys are consecutive words: one store).
      static_assert(US <= SLPR, "one summed row per lane group of SLPR / US lanes");
      const float ssum = transposed_group_sum<US, SLPR>(sc);
      const uint32_t tag = launch_tag(ep);
      if (col % (SLPR / US) == 0) {
        const int64_t c = base + grp + SRPL * (col / (SLPR / US));
        if (c < c1 && c < C) {
          const uint32_t key = order_key(ssum * a.score_scale);
          if (P > 1) {
            if (!mute) put_tagged(kg + c, tag, key);
          } else {
            keys_l[c] = key;
          }
        }
      }
    };
    if (!PIPE || c1 - c0 <= kScoreStride) {
      // Batch by batch: the rows, then q -- the newest load, so waiting for it
      // covers them all: one round trip per batch (one batch per wavefront in
      // the latency-bound shapes; with two workgroups on a CU, one waits while
      // the other computes).  The first batch is requested before the loop,
      // so that what the compiler hoists into the loop's preheader (the key
      // words' address and other non-preloaded arguments, with the wait for
      // their loads) comes after it.
      if (c0 < c1) {
        uint4 rs[US];
        issue_rows(c0, rs);
        uint4 q4 = load_q4();
        for (int64_t blk = c0;;) {
          score_rows(blk, rs, q4);
          blk += kScoreStride;
          if (blk >= c1) break;
          issue_rows(blk, rs);
          q4 = load_q4();
        }
      }
    } else {
      // Several batches, double-buffered: batch i + 1 is requested before batch
      // i is scored.  The last batch is scored in a tail of its own, so no load
      // sits under a branch (a join would make the compiler wait for every
      // load in flight) and none is left in flight after the walk (its
      // registers' next use would wait for it; the branches test the
      // workgroup-uniform blk).  The two buffers alternate without a copy (a
      // copy lets the compiler load into the registers of the batch still in
      // flight).  Here c1 - c0 > kScoreStride: at least two batches.
      const uint4 q4 = load_q4();
      uint4 ra[US], rb[US];
      issue_rows(c0, ra);
      for (int64_t blk = c0;;) {
        issue_rows(blk + kScoreStride, rb);
        score_rows(blk, ra, q4);
        blk += kScoreStride;
        if (blk + kScoreStride >= c1) {
          score_rows(blk, rb, q4);
          break;
        }
        issue_rows(blk + kScoreStride, ra);
        score_rows(blk, rb, q4);
        blk += kScoreStride;
        if (blk + kScoreStride >= c1) {
          score_rows(blk, ra, q4);
          break;
        }
      }
    }
  }

  // (A workgroup with no summary rows scored none.)
  if constexpr (!POS) count_from_device();
  CSAHCA_STAMP(1);
  // ---- B: gather the head's keys, top-k -----------------------------------
  const uint32_t tag = launch_tag(epoch);
  // This thread timed out on a partner's word (or the head is poisoned: then
  // nothing is awaited and the output is NaN).
  bool bad = epoch == kPoisonEpoch;
  if (P > 1 && !bad) {
    const uint64_t* kg = a.keys + h * a.key_stride;
    for (int64_t i0 = tid; i0 < C; i0 += NT * B8) {
      uint64_t w[B8];
#pragma unroll
      for (int j = 0; j < B8; ++j) {
        const int64_t i = i0 + j * NT;
        w[j] = i < C ? get_raw(kg + i) : 0;
      }
#pragma unroll
      for (int j = 0; j < B8; ++j) {
        const int64_t i = i0 + j * NT;
        if (i < C) keys_l[i] = wait_tagged(kg + i, w[j], tag, a.status, a.spin_limit, bad);
      }
    }
  }
  __syncthreads();
  CSAHCA_STAMP(2);
  constexpr int kAttendStride = W * RPL * U;
  // Double-buffered walk of a whole head (PIPE, P = 1, C <= 512): the first
  // batch of phase C lies inside the best chunk, which every wavefront finds
  // with one scan of the keys (exactly the top-k's first slot), so its rows
  // are requested before the selection runs and their round trip overlaps it
  // (B32 H8 top-8, iid keys: S8192 20.5 -> 20.0 us, S32768 28.9 -> 28.6 us;
  // at C = 2048 the scan cost more than it hid).  The batch-by-batch
  // instantiation keeps its code unchanged.
  bool early = false;
  AttendRows<U> r_first;
  uint4 q_first;
  if constexpr (PIPE && W == kStepWaves) {
    const int ns = a.topk * a.chunk;  // this workgroup's slots [0, ns) at P = 1
    early = P == 1 && C > 0 && C <= 512 && a.topk > 0 && a.chunk >= kAttendStride && ns > kAttendStride;
    if (early) {
      const int32_t c_first = wave_top1<8>(keys_l, static_cast<int>(C));
      auto first_id = [&](int) { return c_first; };
      auto tok_first = [&](int s, int64_t& tok) {
        return slot_token_of(first_id, s, a.chunk, a.chunk_shift, a.S, tok);
      };
      const int g = lane / LPR, cl = lane % LPR;
      q_first = load_global_u4(q + cl * VEC);
      attend_issue<T, D, U>(r_first, static_cast<const T*>(a.kcache) + h * a.S * D + cl * VEC,
                            static_cast<const T*>(a.vcache) + h * a.S * D + cl * VEC, wave * RPL * U, ns, g,
                            tok_first);
    }
  }
  if (wave == 0) {
    int32_t* io = a.idx_out + h * a.topk;
    const bool write_ids = (p == 0);
    auto emit = [&](int r, int32_t i) {
      sel[r] = i;
      if (write_ids) io[r] = i;
    };
    // Fewer chunks in play than selection slots (device count only): the
    // slots past the count hold -1, which the attention below skips.
    const int kk = static_cast<int>(min<int64_t>(a.topk, C));
    if (kk > 0) wave_topk<TOPK_M>(keys_l, static_cast<int>(C), kk, tk_scratch, hist, skey, sidx, lcount, emit);
    for (int r = kk + lane; r < a.topk; r += kWave) emit(r, -1);
  }
  __syncthreads();
  CSAHCA_STAMP(3);

  // ---- C: attention over this workgroup's slots ---------------------------
  const int nslots = a.topk * a.chunk;
  int s0, s1;  // 32-bit division whenever nslots * P fits (as for the rows of phase A)
  if (static_cast<int64_t>(nslots) * P <= static_cast<int64_t>(UINT32_MAX)) {
    const uint32_t ns = static_cast<uint32_t>(nslots), up = static_cast<uint32_t>(P);
    s0 = static_cast<int>(ns * static_cast<uint32_t>(p) / up);
    s1 = static_cast<int>(ns * static_cast<uint32_t>(p + 1) / up);
  } else {
    s0 = static_cast<int>(static_cast<int64_t>(nslots) * p / P);
    s1 = static_cast<int>(static_cast<int64_t>(nslots) * (p + 1) / P);
  }
  const int grp = lane / LPR, col = lane % LPR;
  const T* qp = q + col * VEC;  // loaded inside attend_block, after the K/V rows
  const T* __restrict__ kb = static_cast<const T*>(a.kcache) + h * a.S * D + col * VEC;
  const T* __restrict__ vb = static_cast<const T*>(a.vcache) + h * a.S * D + col * VEC;
  auto get_id = [&](int cs) { return sel[cs]; };
  auto tok_of = [&](int s, int64_t& tok) {
    return slot_token_of(get_id, s, a.chunk, a.chunk_shift, a.S, tok);
  };
  WaveSoftmax<T, D> st;
  st.init();
  // Batch by batch, or double-buffered when this workgroup has its CU alone.
  if (!PIPE || s1 - s0 <= kAttendStride) {
    for (int blk = s0; blk < s1; blk += kAttendStride)
      attend_block<T, D, U>(st, qp, a.qscale, kb, vb, blk + wave * RPL * U, s1, grp, tok_of);
  } else if (early) {
    attend_pipelined_from<T, D, U>(st, r_first, q_first, a.qscale, kb, vb, s0 + wave * RPL * U, kAttendStride, s1,
                                   grp, tok_of);
  } else {
    attend_pipelined<T, D, U>(st, qp, a.qscale, kb, vb, s0 + wave * RPL * U, kAttendStride, s1, grp, tok_of);
  }
  // Row groups folded transposed: every lane holds, and stores, kKeep of its
  // columns' sums.
  CSAHCA_STAMP(4);
  const int fbase = fold_row_groups_share(st);
  float* cw = comb + wave * (D + 2);
  // A wavefront in which any lane timed out on a key marks its state with a
  // NaN weight, which poisons the head's output below.
  const bool wave_bad = __any(bad);
  if (lane == 0) {
    cw[0] = st.m;
    cw[1] = wave_bad ? __builtin_nanf("") : st.l;
  }
#pragma unroll
  for (int e = 0; e < FoldShare<T, D>::kKeep; ++e) cw[2 + col * VEC + fbase + e] = st.acc[e];
  __syncthreads();
  float M = -INFINITY;
  bool poisoned = false;
#pragma unroll
  for (int w = 0; w < W; ++w) {
    const float lw = comb[w * (D + 2) + 1];
    poisoned = poisoned || lw != lw;
    if (lw > 0.f) M = fmaxf(M, comb[w * (D + 2)]);
  }
  float Lsum = 0.f, A = 0.f;
  const int d = tid;
  if (M != -INFINITY) {
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float lw = comb[w * (D + 2) + 1];
      if (lw > 0.f) {
        const float wt = fast_exp2(comb[w * (D + 2)] - M);
        Lsum = fmaf(wt, lw, Lsum);
        if (d < D) A = fmaf(wt, comb[w * (D + 2) + 2 + d], A);
      }
    }
  }
  if (poisoned) Lsum = __builtin_nanf("");
  T* __restrict__ out = static_cast<T*>(a.out) + h * D;
  if (P == 1) {
    if (d < D) out[d] = from_f32<T>(poisoned ? Lsum : (Lsum > 0.f ? A / Lsum : 0.f));
    CSAHCA_STAMP(6);
    return;
  }

  // ---- D: publish the partial; workgroup 0 of the head merges -------------
  // Workgroup 0 gathers the P tagged partials directly, each word re-read
  // until it carries this launch's tag: no arrival counter, so no atomic round
  // trip between the last partial and the merge.
  uint64_t* pp = a.part + h * a.part_stride + p * static_cast<int64_t>(D + 2);
  const bool mute = h == 0 && p == a.mute_p;  // the test switch of phase A
  if (!mute) {
    if (d < D) put_tagged(pp + 2 + d, tag, __float_as_uint(A));
    if (tid == 0) {
      put_tagged(pp, tag, __float_as_uint(M));
      put_tagged(pp + 1, tag, __float_as_uint(Lsum));
    }
  }
  CSAHCA_STAMP(5);
  if (p != 0) return;
  const uint64_t* ph = a.part + h * a.part_stride;
  if (MERGE == kMergeRegs || (MERGE == kMergeBoth && P <= kRegMergeP)) {
    // Few partials: the thread of column d gathers every acc_j[d] itself, and
    // lane l of each wavefront one of the 16 words (m_j, l_j), j = (l % 16) / 2,
    // which the wavefront shares by lane permutes -- one batch of 9 tagged loads
    // per thread (partials past P re-read partial 0, columns past D re-read
    // column 0; both dropped) -- and forms the weights and its column: no LDS
    // and no barrier.  Partials are combined in the same order and with the
    // same operations as below.
    // Words not yet tagged are re-read all together, one round trip per
    // round; readiness is decided per wavefront (its lanes hold the (m_j, l_j)
    // words every lane needs).  (Measured: 9 loads per thread per round in
    // place of 24 -- every (m_j, l_j) in every thread -- took the B1 H8 S32768
    // step from 10.63 to 10.20 us; a second round kept in flight half a round
    // trip behind the first was slower, 10.37 us.)
    const int dd = d < D ? d : 0;
    const int jm = (lane & 15) >> 1;
    const uint64_t* pml = ph + static_cast<int64_t>(jm < P ? jm : 0) * (D + 2) + (lane & 1);
    constexpr int NW = kRegMergeP + 1;
    auto poll = [&](uint64_t(&w)[NW]) {
#pragma unroll
      for (int j = 0; j < kRegMergeP; ++j) w[j] = get_raw(ph + static_cast<int64_t>(j < P ? j : 0) * (D + 2) + 2 + dd);
      w[kRegMergeP] = get_raw(pml);
    };
    auto ready = [&](const uint64_t(&w)[NW]) {
      bool r = true;
#pragma unroll
      for (int j = 0; j < NW; ++j) r = r && static_cast<uint32_t>(w[j] >> 32) == tag;
      return __all(r) != 0;
    };
    // Wavefronts past the last column have nothing to merge (wavefront 0, which
    // publishes the epoch, always has columns).
    if (wave * kWave >= D) return;
    // A key that timed out anywhere in the wavefront poisons its columns: no wait.
    if (__any(bad)) bad = true;
    uint64_t wf[NW];
    poll(wf);
    for (uint32_t it = 0;; ++it) {
      if (bad || ready(wf)) break;
      if (it >= a.spin_limit) {
        __hip_atomic_fetch_or(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bad = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      poll(wf);
    }
    float mj[kRegMergeP], lj[kRegMergeP], aj[kRegMergeP];
    const uint32_t mlv = static_cast<uint32_t>(wf[kRegMergeP]);
#pragma unroll
    for (int j = 0; j < kRegMergeP; ++j) {
      mj[j] = __uint_as_float(static_cast<uint32_t>(__shfl(static_cast<int>(mlv), 2 * j, kWave)));
      lj[j] = __uint_as_float(static_cast<uint32_t>(__shfl(static_cast<int>(mlv), 2 * j + 1, kWave)));
      aj[j] = __uint_as_float(static_cast<uint32_t>(wf[j]));
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRegMergeP; ++j) {
      if (j < P && lj[j] > 0.f) mx = fmaxf(mx, mj[j]);
      bad = bad || (j < P && lj[j] != lj[j]);  // a poisoned partial
    }
    float LL = 0.f, AA = 0.f;
#pragma unroll
    for (int j = 0; j < kRegMergeP; ++j) {
      const float w = (j < P && lj[j] > 0.f && mx != -INFINITY) ? fast_exp2(mj[j] - mx) : 0.f;
      LL = fmaf(w, lj[j], LL);
      AA = fmaf(w, aj[j], AA);
    }
    if (d < D) out[d] = from_f32<T>(bad ? __builtin_nanf("") : (LL > 0.f ? AA / LL : 0.f));
    CSAHCA_STAMP(6);
    // Every workgroup of the head has published, so each read this launch's
    // epoch long ago: the next launch's tags can start.  After a time-out (or
    // on a poisoned head) the head is poisoned.
    if (tid == 0)
      __hip_atomic_store(&a.epoch[h], bad ? kPoisonEpoch : tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if constexpr (MERGE != kMergeRegs) {
    // Gather all P partials ((m, l, acc[D]) each) into LDS in one batch of loads
    // spread over the 256 threads, then merge from LDS.
    float* pb = reinterpret_cast<float*>(keys_l);
    const int nw = P * (D + 2);
    for (int i0 = bad ? nw : tid; i0 < nw; i0 += NT * kGather) {
      uint64_t w[kGather];
  #pragma unroll
      for (int j = 0; j < kGather; ++j) {
        const int i = i0 + j * NT;
        w[j] = i < nw ? get_raw(ph + i) : 0;
      }
      bool lost = false;
      wait_tagged_batch<kGather>([&](int j) { return ph + i0 + j * NT; }, [&](int j) { return i0 + j * NT < nw; }, w,
                                 tag, a.status, a.spin_limit, lost);
  #pragma unroll
      for (int j = 0; j < kGather; ++j) {
        const int i = i0 + j * NT;
        // a lost word poisons what uses it
        if (i < nw)
          pb[i] = static_cast<uint32_t>(w[j] >> 32) != tag ? __builtin_nanf("")
                                                           : __uint_as_float(static_cast<uint32_t>(w[j]));
      }
    }
    __syncthreads();
    // Wavefront 0: one partial per lane -> weights 2^(m_j - M) (0 for empty
    // partials) and the total L (NaN if any partial is poisoned); then every
    // column is a branch-free dot product.
    float* wts = comb;  // P weights, then L at [kStepMaxP]
    if (wave == 0) {
      const float mj = lane < P ? pb[lane * (D + 2)] : -INFINITY;
      const float lj = lane < P ? pb[lane * (D + 2) + 1] : 0.f;
      float mx = lj > 0.f ? mj : -INFINITY;
  #pragma unroll
      for (int off = 32; off >= 1; off >>= 1) mx = fmaxf(mx, xor_lanes(mx, off));
      const float w = (lj > 0.f && mx != -INFINITY) ? fast_exp2(mj - mx) : 0.f;
      if (lane < P) wts[lane] = w;
      const float Lt = wave_sum(w * lj);
      const bool any_bad = __any(bad || mj != mj || lj != lj);
      if (lane == 0) wts[kStepMaxP] = any_bad ? __builtin_nanf("") : Lt;
    }
    __syncthreads();
    const float LL = wts[kStepMaxP];
    if (d < D) {
      float AA = 0.f;
  #pragma unroll 8
      for (int j = 0; j < P; ++j) AA = fmaf(wts[j], pb[j * (D + 2) + 2 + d], AA);
      out[d] = from_f32<T>(LL != LL ? LL : (LL > 0.f ? AA / LL : 0.f));
    }
    CSAHCA_STAMP(6);
    __syncthreads();
    // A lost or poisoned partial poisons the head (see the register merge above).
    if (tid == 0)
      __hip_atomic_store(&a.epoch[h], LL != LL ? kPoisonEpoch : tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Every argument of the step, requested from the kernel-argument segment in
// one batch at entry.  Left to itself the compiler loads each argument where
// it is first used: the head/workgroup division waited for one scalar load,
// the pointers of phase A for a second one issued after it -- two dependent
// round trips before the first summary load.
__device__ __forceinline__ void step_args_at_entry(const StepParams& a) {
  asm volatile("" ::"s"(a.q), "s"(a.summary), "s"(a.kcache), "s"(a.vcache), "s"(a.out), "s"(a.idx_out),
               "s"(a.status), "s"(a.epoch), "s"(a.keys), "s"(a.part), "s"(a.key_stride), "s"(a.part_stride));
  asm volatile("" ::"s"(a.S), "s"(a.C), "s"(a.Cs), "s"(a.c_dev), "s"(a.pos_dev), "s"(a.summary_out),
               "s"(a.chunk), "s"(a.chunk_shift), "s"(a.topk), "s"(a.P), "s"(a.colo_bh), "s"(a.score_scale),
               "s"(a.qscale), "s"(a.spin_limit), "s"(a.mute_p));
}

// The arguments phase A needs first also lead the kernel's parameter list as
// scalars (StepLead), which the library is built to preload into SGPRs at
// wave launch (-amdgpu-kernarg-preload-count): the summary and q addresses
// and the epoch word are requested without waiting for any argument load.
struct StepLead {
  const float* summary;
  const void* q;
  uint32_t* epoch;
  int64_t Cs;
  const int32_t* c_dev;
  const int64_t* pos_dev;
  uint32_t colo_bh;
  int32_t P;
};

__host__ __device__ inline StepLead step_lead_of(const StepParams& a) {
  return StepLead{a.summary, a.q, a.epoch, a.Cs, a.c_dev, a.pos_dev, a.colo_bh, a.P};
}

template <typename T, int D, int TOPK_M, bool POS, bool PIPE = false, int W = kStepWaves, int MERGE = kMergeBoth>
__global__ __launch_bounds__(W * kWave) void csa_step_kernel(const float* summary, const void* q, uint32_t* epoch,
                                                             int64_t Cs, const int32_t* c_dev,
                                                             const int64_t* pos_dev, uint32_t colo_bh, int32_t P,
                                                             StepParams a) {
  a.summary = summary;
  a.q = q;
  a.epoch = epoch;
  a.Cs = Cs;
  a.c_dev = c_dev;
  a.pos_dev = pos_dev;
  a.colo_bh = colo_bh;
  a.P = P;
  csa_step_body<T, D, TOPK_M, POS, PIPE, W, MERGE>(a, blockIdx.x);
}

// The hybrid step: blocks [0, step_blocks) run the decode step above, the rest
// the HCA chunk pass over per_block consecutive chunk items each.  The two are
// independent until the HCA merge (a later launch, which also blends), so the
// latency-bound step runs beside the bandwidth-bound chunk stream.  Step blocks
// come first: they wait only on each other, and they are dispatched first.
struct HcaPart {
  const void* q;
  const void* k;
  const void* v;
  float* scores;
  float* means;
  int64_t S;
  int64_t C;
  int64_t items;
  int chunk;
  int per_block;
  float scale;
};

template <typename T, int D, int TOPK_M>
__global__ __launch_bounds__(kStepThreads) void csa_hybrid_kernel(StepParams a, HcaPart hp, uint32_t step_blocks) {
  static_assert(kStepThreads == kHcaThreads, "one block size for both parts");
  if (blockIdx.x < step_blocks) {
    csa_step_body<T, D, TOPK_M, false>(a, blockIdx.x);
    return;
  }
  const int64_t j0 = static_cast<int64_t>(blockIdx.x - step_blocks) * hp.per_block;
  for (int i = 0; i < hp.per_block; ++i) {
    const int64_t item = j0 + i;
    if (item >= hp.items) return;
    if (i > 0) __syncthreads();  // the previous item's LDS reads are done
    hca_chunk_body<T, true>(static_cast<const T*>(hp.q), static_cast<const T*>(hp.k), static_cast<const T*>(hp.v),
                            hp.scores, hp.means, hp.S, D, hp.chunk, hp.C, hp.scale, item);
  }
}

size_t align256(size_t n) { return (n + 255) & ~size_t{255}; }

struct StepLayout {
  size_t epoch, keys, part, total;
};

StepLayout step_layout(int64_t bh, int64_t C, int64_t D, int64_t k, int64_t chunk) {
  StepLayout L;
  L.epoch = 256;
  L.keys = L.epoch + align256(static_cast<size_t>(bh) * 4);
  L.part = L.keys + align256(static_cast<size_t>(bh * C) * 8);
  const size_t fused = static_cast<size_t>(bh * kStepMaxP * (D + 2)) * 8;
  const int64_t tile = csahca_csa_auto_tile_size(1, bh, k, chunk);
  const int64_t tiles = std::max<int64_t>(1, ceil_div(k * chunk, tile));
  const size_t split = align256(static_cast<size_t>(bh * tiles * 2) * 4) + static_cast<size_t>(bh * tiles * D) * 4;
  L.total = L.part + std::max(fused, split);
  return L;
}

// CSAHCA_STEP_WGS_PER_HEAD=n (> 0) overrides the workgroups per head (read per
// call; still bounded by the residency rule of decode_step_impl).
int64_t env_wgs_per_head() {
  const char* s = std::getenv("CSAHCA_STEP_WGS_PER_HEAD");
  return s ? std::max<int64_t>(0, std::atoll(s)) : 0;
}

using StepKernelFn = void (*)(const float*, const void*, uint32_t*, int64_t, const int32_t*, const int64_t*, uint32_t,
                              int32_t, StepParams);
using HybridKernelFn = void (*)(StepParams, HcaPart, uint32_t);

// The instantiation of the step kernel a call launches (m: top-k register rows).
// (lds: the instantiation with the LDS merge, for P > kRegMergeP)
template <typename T, int MG>
StepKernelFn step_kernel_merge(int64_t head_dim, int m, bool pos) {
#define CSAHCA_PICK(DD)                                                                                \
  if (m == 8)                                                                                          \
    return pos ? csa_step_kernel<T, DD, 8, true, false, kStepWaves, MG>                               \
               : csa_step_kernel<T, DD, 8, false, false, kStepWaves, MG>;                             \
  if (m == 32)                                                                                         \
    return pos ? csa_step_kernel<T, DD, 32, true, false, kStepWaves, MG>                              \
               : csa_step_kernel<T, DD, 32, false, false, kStepWaves, MG>;                            \
  return pos ? csa_step_kernel<T, DD, 0, true, false, kStepWaves, MG>                                 \
             : csa_step_kernel<T, DD, 0, false, false, kStepWaves, MG>;
  if (head_dim == 64) { CSAHCA_PICK(64) }
  if (head_dim == 128) { CSAHCA_PICK(128) }
  CSAHCA_PICK(256)
#undef CSAHCA_PICK
}

template <typename T>
StepKernelFn step_kernel_for(int64_t head_dim, int m, bool pos, bool lds) {
  return lds ? step_kernel_merge<T, kMergeLds>(head_dim, m, pos) : step_kernel_merge<T, kMergeRegs>(head_dim, m, pos);
}

StepKernelFn step_kernel_for_dtype(int dtype, int64_t head_dim, int m, bool pos, bool lds) {
  switch (dtype) {
    case CSAHCA_BF16: return step_kernel_for<bf16>(head_dim, m, pos, lds);
    case CSAHCA_F16: return step_kernel_for<f16>(head_dim, m, pos, lds);
    case CSAHCA_F32: return step_kernel_for<float>(head_dim, m, pos, lds);
    default: return nullptr;
  }
}

// The double-buffered instantiation, for a grid with at most one workgroup
// per CU (no neighbour to overlap a workgroup's memory waits with; measured:
// B32 top-8 4-8% faster, and ~1% slower where two workgroups share a CU).
// bf16/f16, head_dim 128, count modes; nullptr elsewhere.
StepKernelFn step_kernel_pipelined(int dtype, int64_t head_dim, int m) {
  if (head_dim != 128) return nullptr;
  if (dtype == CSAHCA_BF16)
    return m == 8 ? csa_step_kernel<bf16, 128, 8, false, true>
                  : m == 32 ? csa_step_kernel<bf16, 128, 32, false, true> : csa_step_kernel<bf16, 128, 0, false, true>;
  if (dtype == CSAHCA_F16)
    return m == 8 ? csa_step_kernel<f16, 128, 8, false, true>
                  : m == 32 ? csa_step_kernel<f16, 128, 32, false, true> : csa_step_kernel<f16, 128, 0, false, true>;
  return nullptr;
}

// The wide instantiation: a head's whole step in one workgroup of
// kWideWaves wavefronts (P = 1, so nothing crosses workgroups and no merge
// beyond the workgroup's own is compiled in), its summary and
// K/V batches double-buffered.  bf16/f16, head_dim 128, count modes; nullptr
// elsewhere.  (8 wavefronts: at 256 heads with top-32 selections 1-4% faster
// than 16, whose extra loads in flight one CU cannot return any faster.)
constexpr int kWideWaves = 8;
StepKernelFn step_kernel_wide(int dtype, int64_t head_dim, int m) {
  if (head_dim != 128) return nullptr;
  if (dtype == CSAHCA_BF16)
    return m == 8    ? csa_step_kernel<bf16, 128, 8, false, true, kWideWaves, kMergeRegs>
           : m == 32 ? csa_step_kernel<bf16, 128, 32, false, true, kWideWaves, kMergeRegs>
                     : csa_step_kernel<bf16, 128, 0, false, true, kWideWaves, kMergeRegs>;
  if (dtype == CSAHCA_F16)
    return m == 8    ? csa_step_kernel<f16, 128, 8, false, true, kWideWaves, kMergeRegs>
           : m == 32 ? csa_step_kernel<f16, 128, 32, false, true, kWideWaves, kMergeRegs>
                     : csa_step_kernel<f16, 128, 0, false, true, kWideWaves, kMergeRegs>;
  return nullptr;
}

// CSAHCA_STEP_WIDE=0 / 1 turns the wide instantiation off / on wherever it
// applies (read per call); unset (-1): the measured rule of decode_step_impl.
int env_step_wide() {
  const char* s = std::getenv("CSAHCA_STEP_WIDE");
  return s ? (std::atoi(s) != 0 ? 1 : 0) : -1;
}

// CSAHCA_STEP_COLOCATE=0 / 1 turns the one-XCD placement of a head's
// workgroups off / on (read per call); unset (-1): the rule of decode_step_impl.
int env_step_colocate() {
  const char* s = std::getenv("CSAHCA_STEP_COLOCATE");
  return s ? (std::atoi(s) != 0 ? 1 : 0) : -1;
}

// CSAHCA_STEP_TEST_TIMEOUT=n (> 0), a test switch for the exchange's
// time-out path (read per call): in a launch with P > 1 the last workgroup of
// head 0 publishes neither keys nor partial, and every bounded wait gives up
// after n polls, so head 0's partners time out -- status bit set, head 0's
// output NaN, head 0 poisoned -- while every workgroup still exits.  0 / unset:
// off.
uint32_t env_step_test_timeout() {
  const char* s = std::getenv("CSAHCA_STEP_TEST_TIMEOUT");
  if (s == nullptr) return 0;
  const long long n = std::atoll(s);
  return n > 0 ? static_cast<uint32_t>(std::min<long long>(n, kSpinLimit)) : 0;
}

HybridKernelFn hybrid_kernel_for(int dtype, int m) {
  if (dtype == CSAHCA_BF16)
    return m == 8 ? csa_hybrid_kernel<bf16, 128, 8> : m == 32 ? csa_hybrid_kernel<bf16, 128, 32>
                                                               : csa_hybrid_kernel<bf16, 128, 0>;
  return m == 8 ? csa_hybrid_kernel<f16, 128, 8> : m == 32 ? csa_hybrid_kernel<f16, 128, 32>
                                                            : csa_hybrid_kernel<f16, 128, 0>;
}

// Workgroups of kernel `fn` (kStepThreads threads, `lds` bytes of dynamic LDS)
// that one CU holds at once, from the occupancy API; cached per device, kernel
// and LDS size.  0 if the query fails.
int resident_per_cu(const void* fn, size_t lds) {
  struct Entry {
    int dev;
    const void* fn;
    size_t lds;
    int n;
  };
  static std::mutex mu;
  static std::vector<Entry> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  {
    std::lock_guard<std::mutex> g(mu);
    for (const Entry& e : cache)
      if (e.dev == dev && e.fn == fn && e.lds == lds) return e.n;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, kStepThreads, lds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  std::lock_guard<std::mutex> g(mu);
  if (cache.size() < 4096) cache.push_back({dev, fn, lds, n});
  return n;
}

// Where a step launch keeps its exchange state: carved from the caller's
// workspace (strides 0: the call's chunk count and P * (head_dim + 2)), or a
// fixed per-head layout that does not depend on the call's shape.
struct StepRegions {
  uint32_t* status;
  uint32_t* epoch;
  uint64_t* keys;
  uint64_t* part;
  int64_t key_stride;   // words per head; 0 = the call's chunk count
  int64_t part_stride;  // words per head; 0 = P * (head_dim + 2)
  int64_t max_p;        // most workgroups per head the partial region holds
};

}  // namespace
}  // namespace csahca

using namespace csahca;

extern "C" size_t csahca_csa_step_workspace_bytes(int64_t batch, int64_t heads, int64_t num_chunks,
                                                  int64_t head_dim, int64_t top_k,
                                                  int64_t chunk_size) {
  if (batch < 0 || heads < 0 || num_chunks < 0 || head_dim < 0 || top_k < 0 || chunk_size <= 0) return 0;
  const int64_t k = std::min(top_k, num_chunks);
  return step_layout(batch * heads, num_chunks, head_dim, k, chunk_size).total;
}

namespace {

// One decode step over num_chunks summary rows per head; with c_dev set the
// chunks in play are *c_dev (clamped to [0, num_chunks]), read on the device.
int decode_step_impl(const void* q, const void* k_cache, const void* v_cache, const float* summary, void* out,
                     int32_t* out_indices, int dtype, int64_t batch, int64_t heads, int64_t seq_len,
                     int64_t head_dim, int64_t num_chunks, const int32_t* c_dev, const int64_t* pos_dev,
                     int64_t chunk_size, int64_t top_k, void* workspace, size_t workspace_bytes,
                     void* stream_ptr, HcaPart* hybrid = nullptr, size_t hybrid_lds = 0,
                     bool* hybrid_launched = nullptr, const StepRegions* fixed = nullptr) {
  CSAHCA_REQUIRE(valid_dtype(dtype), "q, k_cache and v_cache must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(batch >= 0 && heads >= 0 && seq_len >= 0 && head_dim >= 0 && num_chunks >= 0,
                 "negative dimension");
  CSAHCA_REQUIRE(chunk_size > 0 && chunk_size <= INT_MAX, "chunk_size must be positive");
  CSAHCA_REQUIRE(top_k >= 0, "top_k must be non-negative");
  CSAHCA_REQUIRE(head_dim <= 1024, "head_dim > 1024 is not supported");
  CSAHCA_REQUIRE(num_chunks <= INT_MAX && num_chunks * chunk_size <= seq_len,
                 "summaries cover more chunks than the cache holds");
  const int64_t k = std::min(top_k, num_chunks);
  CSAHCA_REQUIRE(k <= 4096, "top_k > 4096 is not supported by the selection kernel");
  CSAHCA_REQUIRE(k * chunk_size <= INT_MAX, "top_k * chunk_size must fit in int32");
  const int64_t bh = batch * heads;
  if (bh == 0 || head_dim == 0) return CSAHCA_OK;
  CSAHCA_REQUIRE(q && out && summary && (k == 0 || (k_cache && v_cache && out_indices)),
                 "null tensor pointer");
  StepLayout lay{};
  char* ws = static_cast<char*>(workspace);
  StepRegions rg{};
  if (fixed == nullptr) {
    lay = step_layout(bh, num_chunks, head_dim, k, chunk_size);
    if (workspace == nullptr || workspace_bytes < lay.total)
      return fail(CSAHCA_ERR_WORKSPACE, "workspace too small for csa decode step");
    rg = StepRegions{reinterpret_cast<uint32_t*>(ws), reinterpret_cast<uint32_t*>(ws + lay.epoch),
                     reinterpret_cast<uint64_t*>(ws + lay.keys), reinterpret_cast<uint64_t*>(ws + lay.part), 0, 0,
                     kStepMaxP};
  } else {
    rg = *fixed;
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);

  const int ncu = device_cu_count();
  const bool aligned = ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_cache) |
                         reinterpret_cast<uintptr_t>(v_cache) | reinterpret_cast<uintptr_t>(summary)) %
                        16) == 0;
  const bool fused_dtype = dtype == CSAHCA_BF16 || dtype == CSAHCA_F16 || dtype == CSAHCA_F32;
  const bool fused_dim = head_dim == 64 || head_dim == 128 || head_dim == 256;
  // One wide workgroup (8 wavefronts) per head where the grid holds about one
  // head per CU and a head selects more than 1024 rows: there the split kernel
  // would take P = 2 and its exchange, while 8 wavefronts keep more of the
  // head's loads in flight (measured at 256 heads, top-32 of 64-token chunks:
  // 3-5% faster).  With fewer heads the split kernel is faster: one CU
  // returns about 64 B per clock to its wavefronts, so a head read through
  // one CU takes ~4 us per 256 KiB, where P workgroups share it.
  const int wide_env = env_step_wide();
  const bool wide_ok = k > 0 && k <= kStepMaxK && (dtype == CSAHCA_BF16 || dtype == CSAHCA_F16) &&
                       head_dim == 128 && aligned && ncu > 0 && pos_dev == nullptr && hybrid == nullptr &&
                       env_wgs_per_head() == 0;
  const bool wide = wide_ok && (wide_env >= 0 ? wide_env == 1
                                              : (bh <= ncu && 2 * bh > ncu && k * chunk_size > 1024));
  const int waves = wide ? kWideWaves : kStepWaves;
  const size_t lds_base = kCandBytes + (256 + 3 * static_cast<size_t>(k) + 1) * 4 +
                          static_cast<size_t>(waves * (head_dim + 2)) * 4;
  // Workgroups per head: the smallest P at which every wavefront streams its
  // share of summary rows and of selected K/V rows in ONE batch of loads (a
  // dependent HBM round trip, ~1.5 us, costs more than the cross-workgroup
  // exchange a larger P adds), capped at ~2 workgroups per CU over the grid.
  int64_t P = wide ? 1 : env_wgs_per_head();
  if (P == 0 && ncu > 0) {
    const int64_t esz = dtype == CSAHCA_F32 ? 4 : 2;
    const int64_t score_rows = int64_t{kStepWaves} * kStepScoreUnroll * std::max<int64_t>(1, kWave / (head_dim / 4));
    const int64_t attend_rows =
        int64_t{kStepWaves} * kStepAttendUnroll * std::max<int64_t>(1, kWave / (head_dim / (16 / esz)));
    P = std::max(ceil_div(num_chunks, score_rows), ceil_div(k * chunk_size, attend_rows));
    P = std::min<int64_t>(P, std::max<int64_t>(1, (2 * static_cast<int64_t>(ncu)) / std::max<int64_t>(bh, 1)));
    // With a head per CU already, splitting a head pays only when its selected
    // rows are many: at 256 heads, P = 1 beats P = 2 by 8-11% with 512 rows
    // (top-8 of 64) and loses by 6% with 2048 (top-32).
    if (bh >= ncu && k * chunk_size <= 1024) P = 1;
    // Above 16 workgroups per head, where half as many still leave each
    // workgroup a CU of its own and the double-buffered instantiation runs
    // (bf16/f16, head_dim 128, no position mode, not the hybrid), half as many
    // workgroups walking two batches each beat the one-batch split: the key
    // exchange and the merge shrink with P.  Measured at B1 H8, P 32 -> 16:
    // S32768 top-32 14.0 -> 13.1 us, S131072 top-8 15.0 -> 14.8, top-32
    // 16.7 -> 16.6; S8192 top-32 level.
    const bool pipe_ok = (dtype == CSAHCA_BF16 || dtype == CSAHCA_F16) && head_dim == 128 && pos_dev == nullptr &&
                         hybrid == nullptr;
    if (P > 16 && pipe_ok && bh * (P / 2) <= ncu) P /= 2;
  }
  P = std::min<int64_t>({P, rg.max_p, ceil_div(num_chunks, 8), ceil_div(k * chunk_size, 16)});
  P = std::max<int64_t>(1, P);
  // keys region (first, its size rounded to 16 bytes): the head's C keys,
  // later (P > 1) the P gathered partials
  auto lds_for = [&](int64_t np) {
    const int64_t words = std::max<int64_t>(num_chunks, np > 1 ? np * (head_dim + 2) : 0);
    return lds_base + static_cast<size_t>((words + 3) & ~int64_t{3}) * 4;
  };
  size_t lds = lds_for(P);
  if (k > 0 && k <= kStepMaxK && fused_dtype && fused_dim && aligned && ncu > 0 && lds <= kStepLds) {
    const int m = topk_regs_for(num_chunks, k);
    const bool hyb = hybrid != nullptr && head_dim == 128 && pos_dev == nullptr &&
                     (dtype == CSAHCA_BF16 || dtype == CSAHCA_F16);
    const HybridKernelFn hfn = hyb ? hybrid_kernel_for(dtype, m) : nullptr;
    // (the step kernel with the merge P needs: from registers up to
    // kRegMergeP partials, through LDS beyond)
    auto step_fn = [&] { return step_kernel_for_dtype(dtype, head_dim, m, pos_dev != nullptr, P > kRegMergeP); };
    StepKernelFn sfn = hyb ? nullptr : step_fn();
    auto launch_lds = [&] { return hyb ? std::max(lds, hybrid_lds) : lds; };
    // The P workgroups of a head wait on each other, so with P > 1 every step
    // workgroup of the grid must fit on the device at once (measured for the
    // instantiation launched, with its LDS); the step blocks of the hybrid
    // kernel come first in its grid.  Where they would not fit, P shrinks,
    // down to 1 (no exchange at all), and the kernel is picked again for the
    // new P (and checked again).
    for (int pass = 0; P > 1 && pass < 4; ++pass) {
      const void* fn = hyb ? reinterpret_cast<const void*>(hfn) : reinterpret_cast<const void*>(sfn);
      const int64_t cap = static_cast<int64_t>(resident_per_cu(fn, launch_lds())) * ncu;
      if (bh * P <= cap) break;
      P = cap / bh;
      if (P < 2) P = 1;
      lds = lds_for(P);
      if (!hyb) sfn = step_fn();
    }
    CSAHCA_REQUIRE(bh * P <= INT32_MAX, "too many heads in one call");
    StepParams pr;
    pr.q = q;
    pr.summary = summary;
    pr.kcache = k_cache;
    pr.vcache = v_cache;
    pr.out = out;
    pr.idx_out = out_indices;
    pr.status = rg.status;
    pr.epoch = rg.epoch;
    pr.keys = rg.keys;
    pr.part = rg.part;
    pr.key_stride = rg.key_stride > 0 ? rg.key_stride : num_chunks;
    pr.part_stride = rg.part_stride > 0 ? rg.part_stride : P * (head_dim + 2);
    pr.S = seq_len;
    pr.C = num_chunks;
    pr.Cs = num_chunks;
    pr.c_dev = c_dev;
    pr.pos_dev = pos_dev;
    pr.summary_out = const_cast<float*>(summary);
    pr.chunk = static_cast<int>(chunk_size);
    int shift = -1;
    if ((chunk_size & (chunk_size - 1)) == 0) {
      shift = 0;
      while ((int64_t{1} << shift) < chunk_size) ++shift;
    }
    pr.chunk_shift = shift;
    pr.topk = static_cast<int>(k);
    pr.P = static_cast<int>(P);
    // A head's workgroups on one XCD (workgroups go to XCD blockIdx % 8):
    // block b serves head b % (B*H), so with B*H a multiple of 8 the P
    // workgroups of a head share an XCD and its L2.  By default only with
    // one head per XCD (B*H = 8) and not in the hybrid launch (measured, graph
    // period at 2048 steps: B1 H8 S32768 top-8 10.55 -> 10.32 us; at 64 heads
    // 0.4-1.1 us slower, the hybrid step ~0.8 us slower, 256 heads level).
    const int colo_env = env_step_colocate();
    const bool colo = P > 1 && (colo_env >= 0 ? colo_env == 1 : (bh == 8 && !hyb));
    pr.colo_bh = colo ? static_cast<uint32_t>(bh) : 0u;
    pr.score_scale = 1.0f / sqrtf(static_cast<float>(head_dim));
    pr.qscale = kLog2e / sqrtf(static_cast<float>(head_dim));
    // Test switch for the time-out path: the last workgroup of head 0 publishes
    // nothing, and every wait gives up after the given number of polls.
    const uint32_t test_polls = env_step_test_timeout();
    pr.spin_limit = test_polls > 0 ? test_polls : kSpinLimit;
    pr.mute_p = (test_polls > 0 && P > 1) ? static_cast<int32_t>(P - 1) : -1;
    if (hyb) {
      const int64_t hblocks = ceil_div(hybrid->items, static_cast<int64_t>(hybrid->per_block));
      CSAHCA_REQUIRE(bh * P + hblocks <= INT32_MAX, "too many blocks in one call");
      *hybrid_launched = true;
      return launch("csa_hybrid_kernel", hfn, dim3(static_cast<uint32_t>(bh * P + hblocks)), dim3(kStepThreads),
                    launch_lds(), stream, pr, *hybrid, static_cast<uint32_t>(bh * P));
    }
    if (wide) {
      const StepKernelFn wf = step_kernel_wide(dtype, head_dim, m);
      const StepLead ld = step_lead_of(pr);
      return launch("csa_step_kernel", wf, dim3(static_cast<uint32_t>(bh)), dim3(kWideWaves * kWave), lds, stream,
                    ld.summary, ld.q, ld.epoch, ld.Cs, ld.c_dev, ld.pos_dev, ld.colo_bh, ld.P, pr);
    }
    StepKernelFn run = sfn;
    // (only where some wavefront has more than one batch of rows to walk)
    const int64_t score_batch = int64_t{kStepWaves} * kStepScoreUnroll * (kWave / (head_dim / 4));
    const int64_t attend_batch = int64_t{kStepWaves} * kStepAttendUnroll * (kWave / (head_dim / (16 / 2)));
    const bool batches = ceil_div(num_chunks, P) > score_batch || ceil_div(k * chunk_size, P) > attend_batch;
    if (pos_dev == nullptr && bh * P <= ncu && batches) {
      if (const StepKernelFn pf = step_kernel_pipelined(dtype, head_dim, m)) run = pf;
    }
    const StepLead ld = step_lead_of(pr);
    return launch("csa_step_kernel", run, dim3(static_cast<uint32_t>(bh * P)), dim3(kStepThreads), lds, stream,
                  ld.summary, ld.q, ld.epoch, ld.Cs, ld.c_dev, ld.pos_dev, ld.colo_bh, ld.P, pr);
  }
  if (fixed != nullptr)
    return fail(CSAHCA_ERR_ARGUMENT,
                "the allocation-free step takes float32/float16/bfloat16, head_dim 64/128/256, 16-byte aligned "
                "tensors and 0 < top_k <= 1024");
  if (c_dev != nullptr || pos_dev != nullptr)
    return fail(CSAHCA_ERR_ARGUMENT,
                "a device chunk count needs the fused step (float32/float16/bfloat16, head_dim 64/128/256, "
                "16-byte aligned tensors, top_k <= 1024)");
  // General path: score + top-k kernels, then the split-KV decode.
  uint32_t* keys = reinterpret_cast<uint32_t*>(ws + lay.keys);
  if (k > 0) {
    int rc = csa_select_launch(q, summary, out_indices, dtype, bh, num_chunks, head_dim, k, keys, stream);
    if (rc != CSAHCA_OK) return rc;
  }
  const int64_t tile = csahca_csa_auto_tile_size(batch, heads, k, chunk_size);
  return csahca_csa_decode_forward_tiled(q, k_cache, v_cache, out_indices, out, dtype, CSAHCA_I32, batch,
                                         heads, seq_len, head_dim, k, chunk_size, tile, ws + lay.part,
                                         lay.total - lay.part, stream);
}

}  // namespace

extern "C" int csahca_csa_decode_step(const void* q, const void* k_cache, const void* v_cache,
                                      const float* summary, void* out, int32_t* out_indices,
                                      int dtype, int64_t batch, int64_t heads, int64_t seq_len,
                                      int64_t head_dim, int64_t num_chunks, int64_t chunk_size,
                                      int64_t top_k, void* workspace, size_t workspace_bytes,
                                      void* stream_ptr) {
  clear_error();
  return decode_step_impl(q, k_cache, v_cache, summary, out, out_indices, dtype, batch, heads, seq_len, head_dim,
                          num_chunks, nullptr, nullptr, chunk_size, top_k, workspace, workspace_bytes, stream_ptr);
}

extern "C" int csahca_csa_decode_step_dev(const void* q, const void* k_cache, const void* v_cache,
                                          const float* summary, const int32_t* num_chunks_dev, void* out,
                                          int32_t* out_indices, int dtype, int64_t batch, int64_t heads,
                                          int64_t seq_len, int64_t head_dim, int64_t max_chunks,
                                          int64_t chunk_size, int64_t top_k, void* workspace,
                                          size_t workspace_bytes, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(num_chunks_dev != nullptr, "null num_chunks pointer");
  return decode_step_impl(q, k_cache, v_cache, summary, out, out_indices, dtype, batch, heads, seq_len, head_dim,
                          max_chunks, num_chunks_dev, nullptr, chunk_size, top_k, workspace, workspace_bytes,
                          stream_ptr);
}

extern "C" int csahca_csa_decode_step_at(const void* q, const void* k_cache, const void* v_cache, float* summary,
                                         const int64_t* token_pos, void* out, int32_t* out_indices, int dtype,
                                         int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                                         int64_t max_chunks, int64_t chunk_size, int64_t top_k, void* workspace,
                                         size_t workspace_bytes, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(token_pos != nullptr, "null token_pos pointer");
  return decode_step_impl(q, k_cache, v_cache, summary, out, out_indices, dtype, batch, heads, seq_len, head_dim,
                          max_chunks, nullptr, token_pos, chunk_size, top_k, workspace, workspace_bytes,
                          stream_ptr);
}

namespace {
int noalloc_status_word(const void** word);
}

extern "C" int csahca_csa_step_status(const void* workspace, uint32_t* status_out, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(status_out, "null pointer");
  // A null workspace names the allocation-free step's state on the current device.
  if (workspace == nullptr) {
    const int rc = noalloc_status_word(&workspace);
    if (rc != CSAHCA_OK) return rc;
  }
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  hipError_t e = hipMemcpyAsync(status_out, workspace, sizeof(uint32_t), hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess) return fail_hip(e, "csahca_csa_step_status");
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return fail_hip(e, "csahca_csa_step_status");
  return CSAHCA_OK;
}

extern "C" int csahca_hybrid_decode_forward(const void* q, const void* k_cache, const void* v_cache,
                                            const float* summary, void* csa_out, int32_t* csa_indices, void* out,
                                            int dtype, int64_t batch, int64_t heads, int64_t seq_len,
                                            int64_t head_dim, int64_t num_chunks, int64_t csa_chunk_size,
                                            int64_t top_k, int64_t hca_chunk_size, double csa_weight,
                                            void* step_workspace, size_t step_workspace_bytes, void* hca_workspace,
                                            size_t hca_workspace_bytes, void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(valid_dtype(dtype), "q, k_cache and v_cache must be float32, float64, float16 or bfloat16");
  CSAHCA_REQUIRE(batch >= 0 && heads >= 0 && seq_len >= 0 && head_dim >= 0, "negative dimension");
  CSAHCA_REQUIRE(hca_chunk_size > 0 && hca_chunk_size <= INT_MAX, "chunk_size must be positive");
  CSAHCA_REQUIRE(seq_len % hca_chunk_size == 0, "seq length must be divisible by chunk_size");
  const int64_t bh = batch * heads;
  if (bh == 0 || head_dim == 0) return CSAHCA_OK;
  const int64_t Ch = seq_len / hca_chunk_size;
  if (Ch == 0) return fail(CSAHCA_ERR_ARGUMENT, "seq length must be at least chunk_size");
  CSAHCA_REQUIRE(bh * Ch <= INT32_MAX, "too many chunks in one call");
  CSAHCA_REQUIRE(q && k_cache && v_cache && out && csa_out, "null tensor pointer");
  const size_t need = csahca_hca_decode_workspace_bytes(batch, heads, seq_len, head_dim, hca_chunk_size);
  if (hca_workspace == nullptr || hca_workspace_bytes < need)
    return fail(CSAHCA_ERR_WORKSPACE, "workspace too small for hca decode");
  // One launch for the step and the HCA chunk pass where the fused step runs
  // (bf16/f16, head_dim 128, 16-byte aligned K/V); otherwise the two ops in
  // turn.  Each HCA block takes two chunk items, so that with the step's
  // register count the whole grid is resident at once.
  const bool aligned = ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) % 16) == 0;
  HcaPart hp{};
  hp.q = q;
  hp.k = k_cache;
  hp.v = v_cache;
  hp.scores = static_cast<float*>(hca_workspace);
  hp.means = reinterpret_cast<float*>(static_cast<char*>(hca_workspace) + hca_workspace_means_offset(bh * Ch));
  hp.S = seq_len;
  hp.C = Ch;
  hp.items = bh * Ch;
  hp.chunk = static_cast<int>(hca_chunk_size);
  hp.per_block = 2;
  hp.scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(head_dim)));
  // LDS of the chunk pass at head_dim 128, 16-byte rows: 16 row groups of K and V column sums.
  const size_t hca_lds = 2 * static_cast<size_t>(kHcaThreads / (128 / 8)) * 128 * sizeof(float);
  bool fused = false;
  hipStream_t stream = static_cast<hipStream_t>(stream_ptr);
  int rc = decode_step_impl(q, k_cache, v_cache, summary, csa_out, csa_indices, dtype, batch, heads, seq_len,
                            head_dim, num_chunks, nullptr, nullptr, csa_chunk_size, top_k, step_workspace,
                            step_workspace_bytes, stream_ptr, (aligned && head_dim == 128) ? &hp : nullptr,
                            hca_lds, &fused);
  if (rc != CSAHCA_OK) return rc;
  if (!fused)
    return csahca_hca_decode_forward(q, k_cache, v_cache, csa_out, csa_weight, out, dtype, batch, heads, seq_len,
                                     head_dim, hca_chunk_size, hca_workspace, hca_workspace_bytes, stream_ptr);
  return hca_merge_launch(dtype, hca_workspace, csa_out, csa_weight, out, bh, Ch, static_cast<int>(head_dim), stream);
}

// ---------------------------------------------------------------------------
// Allocation-free decode step (csahca_csa_decode_step_noalloc).
//
// The exchange state lives in `scratch`, a static device array: one copy per
// device, zero when the library's code object is loaded on that device, held
// until the process ends.  Its layout does not depend on the call's shape:
// head slot h (h < kFixedHeads) always has its epoch word, kFixedChunks key
// words and kFixedP * (kFixedDim + 2) partial words at the same place, and
// every launch over slot h advances that slot's epoch by one.  Every word left
// in slot h by an earlier call therefore carries an older tag than the
// current launch's, whatever shapes earlier calls had, so nothing is cleared
// between calls.  Calls that overlap on one device (two streams) race on it.
namespace {
constexpr int64_t kFixedHeads = 256;    // batch * heads
constexpr int64_t kFixedChunks = 2048;  // summary rows per head
constexpr int64_t kFixedDim = 256;      // head_dim
constexpr int64_t kFixedP = 32;         // workgroups per head
constexpr int64_t kFixedHeaderWords = 32;                // 256 B: the status word
constexpr int64_t kFixedEpochWords = kFixedHeads / 2;    // one u32 epoch per head slot
constexpr int64_t kFixedKeyWords = kFixedChunks;         // per head slot
constexpr int64_t kFixedPartWords = kFixedP * (kFixedDim + 2);  // per head slot
constexpr int64_t kFixedWords =
    kFixedHeaderWords + kFixedEpochWords + kFixedHeads * (kFixedKeyWords + kFixedPartWords);  // 21.1 MB
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) uint64_t scratch[kFixedWords];

namespace {
std::mutex g_scratch_mu;
uint64_t* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's `scratch` (hipGetSymbolAddress once
// per device, with that device current).  The array's name in host code is a
// stand-in, not a device address: only this pointer goes to kernels.
int scratch_regions(StepRegions* rg) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail_hip(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(CSAHCA_ERR_ARGUMENT, "device ordinal out of range");
  uint64_t* base = nullptr;
  {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    base = g_scratch_ptr[dev];
    if (base == nullptr) {
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return fail_hip(e, "hipGetSymbolAddress(scratch)");
      base = static_cast<uint64_t*>(p);
      g_scratch_ptr[dev] = base;
    }
  }
  rg->status = reinterpret_cast<uint32_t*>(base);
  rg->epoch = reinterpret_cast<uint32_t*>(base + kFixedHeaderWords);
  rg->keys = base + kFixedHeaderWords + kFixedEpochWords;
  rg->part = rg->keys + kFixedHeads * kFixedKeyWords;
  rg->key_stride = kFixedKeyWords;
  rg->part_stride = kFixedPartWords;
  rg->max_p = kFixedP;
  return CSAHCA_OK;
}

int noalloc_status_word(const void** word) {
  StepRegions rg{};
  const int rc = scratch_regions(&rg);
  if (rc != CSAHCA_OK) return rc;
  *word = rg.status;
  return CSAHCA_OK;
}

// Zero-fills `words` 64-bit words (16 bytes per thread per store, grid-stride).
__global__ __launch_bounds__(256) void scratch_zero_kernel(uint64_t* p, int64_t words) {
  const int64_t pairs = words / 2;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  uint4* p4 = reinterpret_cast<uint4*>(p);
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < pairs; i += stride)
    p4[i] = make_uint4(0u, 0u, 0u, 0u);
  if (blockIdx.x == 0 && threadIdx.x == 0 && (words & 1)) p[words - 1] = 0;
}
}  // namespace

extern "C" int csahca_csa_decode_step_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                              const float* summary, void* out, int32_t* out_indices, int dtype,
                                              int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                                              int64_t num_chunks, int64_t chunk_size, int64_t top_k,
                                              void* stream_ptr) {
  clear_error();
  CSAHCA_REQUIRE(batch >= 0 && heads >= 0 && seq_len >= 0 && head_dim >= 0 && num_chunks >= 0,
                 "negative dimension");
  CSAHCA_REQUIRE(batch * heads <= kFixedHeads,
                 "csahca_csa_decode_step_noalloc: batch * heads exceeds 256, the static scratch limit");
  CSAHCA_REQUIRE(num_chunks <= kFixedChunks,
                 "csahca_csa_decode_step_noalloc: num_chunks exceeds 2048, the static scratch limit");
  CSAHCA_REQUIRE(head_dim <= kFixedDim, "csahca_csa_decode_step_noalloc: head_dim exceeds 256");
  CSAHCA_REQUIRE(batch * heads == 0 || head_dim == 0 || (top_k > 0 && num_chunks > 0),
                 "csahca_csa_decode_step_noalloc needs top_k > 0 and at least one chunk");
  StepRegions rg{};
  const int rc = scratch_regions(&rg);
  if (rc != CSAHCA_OK) return rc;
  return decode_step_impl(q, k_cache, v_cache, summary, out, out_indices, dtype, batch, heads, seq_len, head_dim,
                          num_chunks, nullptr, nullptr, chunk_size, top_k, nullptr, 0, stream_ptr, nullptr, 0,
                          nullptr, &rg);
}

// Zero the allocation-free step's state on the current device (status word,
// epochs, keys and partials), on `stream`, with a fill kernel (capturable).
// The caller must order it after every earlier allocation-free call and before
// every later one (the same stream does).  This is how a head slot poisoned by
// an exchange time-out is cleared.
extern "C" int csahca_csa_step_noalloc_reset(void* stream_ptr) {
  clear_error();
  StepRegions rg{};
  const int rc = scratch_regions(&rg);
  if (rc != CSAHCA_OK) return rc;
  uint64_t* base = reinterpret_cast<uint64_t*>(rg.status);
  return launch("scratch_zero_kernel", scratch_zero_kernel, dim3(1024), dim3(256), 0,
                static_cast<hipStream_t>(stream_ptr), base, kFixedWords);
}

#ifdef CSAHCA_STEP_TIMELINE
// The timeline build's extra entry points: copy the stamps of the first
// `blocks` workgroups of the last step launch (blocks x 8 uint64) to host
// memory, zero them, and the stamps' clock rate.
extern "C" int csahca_step_timeline_read(uint64_t* host, int64_t blocks) {
  if (blocks < 0 || blocks > csahca::kTimelineBlocks) return CSAHCA_ERR_ARGUMENT;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(csahca::g_timeline),
                             sizeof(uint64_t) * csahca::kTimelineStamps * static_cast<size_t>(blocks), 0,
                             hipMemcpyDeviceToHost) == hipSuccess
             ? CSAHCA_OK
             : CSAHCA_ERR_HIP;
}

// Frequency of the stamps' clock in kHz (0 if the query fails).
extern "C" int64_t csahca_step_timeline_rate_khz() {
  int dev = 0, khz = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev) != hipSuccess)
    return 0;
  return khz;
}

extern "C" int csahca_step_timeline_clear() {
  static uint64_t zero[csahca::kTimelineBlocks][csahca::kTimelineStamps];
  return hipMemcpyToSymbol(HIP_SYMBOL(csahca::g_timeline), zero, sizeof(zero), 0, hipMemcpyHostToDevice) ==
                 hipSuccess
             ? CSAHCA_OK
             : CSAHCA_ERR_HIP;
}
#endif
