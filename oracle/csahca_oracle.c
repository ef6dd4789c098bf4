/*
 * csahca_oracle.c -- CPU restatement of the CSAHCA reference's decode algorithms.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker that the HIP kernels of
 * csahca_amd are compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path (csahca_amd) never
 * calls it and has no CPU fallback.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference checkout, ypd666/CSAHCA).
 *
 * Arithmetic: inputs arrive as fp32 arrays (exact copies of bf16/f16/f32 data);
 * dot products, softmax and weighted sums run in double; rounding to the storage
 * type happens exactly where the reference rounds (probability cast in
 * torch-csa, summary cast in HCA, bf16 nope cast in the DSV4 dequant).
 *
 * Edge semantics follow the reference KERNELS where the torch oracles are
 * undefined: chunk id < 0 -> slot skipped, token >= seq_len -> skipped
 * (csrc/csa_attention.cu:48-56,179-185); DSV4 slot >= length or index < 0 ->
 * skipped (csrc/dsv4_attention.cu:186-225); no valid token and no sink -> 0
 * (csrc/csa_attention.cu:87, csrc/dsv4_attention.cu:307).  One deliberate
 * extension: a DSV4 location beyond the cache (page >= num_pages) is skipped
 * like a negative one (the reference kernel would read out of bounds).
 *
 * Pinning status (what checks this file):
 *   - e4m3fn encode/decode: exhaustive 256-code table and a dense float sweep
 *     against torch.float8_e4m3fn (tests/test_oracle_formats.py).
 *   - bf16/f16 rounding: dense sweeps against torch casts.
 *   - chunk_mean / select_topk / csa_attend / hca / dsv4 pack, dequant and
 *     attention: golden vectors written by the reference's own Python functions
 *     (tests/golden/), closed forms and planted-chunk known answers
 *     (tests/test_oracle_csa.py, tests/test_oracle_dsv4.py).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

/* Storage types, numbered like csahca_dtype in include/csahca.h. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_BF16 = 2, ORC_F64 = 3 };

/* ------------------------------------------------------------------------ */
/* Scalar format helpers                                                      */
/* ------------------------------------------------------------------------ */

/* Round fp32 to the nearest bfloat16 (ties to even), returned as fp32.
 * torch's Tensor.to(torch.bfloat16) rounding. */
static float round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) {
    if (u & 0x007fffffu) u |= 0x00400000u; /* keep NaN quiet */
    u &= 0xffff0000u;
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
  }
  memcpy(&x, &u, 4);
  return x;
}

/* Round fp32 to the nearest IEEE binary16 (ties to even), returned as fp32. */
static float round_f16(float x) {
  if (isnan(x)) return x;
  float ax = fabsf(x);
  if (ax >= 65520.0f) return copysignf(INFINITY, x);
  float q;
  if (ax < 6.103515625e-05f) {
    q = 5.9604644775390625e-08f; /* 2^-24: subnormal quantum */
  } else {
    int e;
    frexpf(ax, &e);
    q = ldexpf(1.0f, e - 11); /* 11 significant bits */
  }
  return copysignf(rintf(ax / q) * q, x);
}

static float round_to(float x, int dtype) {
  switch (dtype) {
    case ORC_BF16: return round_bf16(x);
    case ORC_F16: return round_f16(x);
    default: return x;
  }
}

/* OCP FP8 E4M3 ("fn": bias 7, max 448, no infinities, NaN = S.1111.111).
 * Decode of one byte -- the __nv_fp8_e4m3 conversion used by
 * csrc/dsv4_attention.cu:21-25 and torch.float8_e4m3fn in
 * hybrid_attention/dsv4_correctness.py:64,76. */
static float e4m3fn_decode(uint8_t b) {
  const int s = b >> 7, e = (b >> 3) & 0xf, m = b & 7;
  float v;
  if (e == 15 && m == 7) {
    v = NAN;
  } else if (e == 0) {
    v = ldexpf((float)m, -9);
  } else {
    v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
  }
  return s ? -v : v;
}

/* Encode with round-to-nearest-even; a magnitude that rounds above 448 becomes
 * NaN (torch's float8_e4m3fn cast: no saturation, no infinity). */
static uint8_t e4m3fn_encode(float x) {
  const uint8_t sign = signbit(x) ? 0x80 : 0;
  if (isnan(x)) return sign | 0x7f;
  const float ax = fabsf(x);
  float r;
  if (ax < 0.015625f) {
    r = rintf(ax * 512.0f) / 512.0f; /* subnormal quantum 2^-9 */
  } else {
    int e;
    frexpf(ax, &e);
    const float q = ldexpf(1.0f, e - 4); /* 4 significant bits */
    r = rintf(ax / q) * q;
  }
  if (!(r <= 448.0f)) return sign | 0x7f;
  if (r == 0.0f) return sign;
  if (r < 0.015625f) return sign | (uint8_t)(int)(r * 512.0f);
  int e;
  const float m = frexpf(r, &e); /* r = m * 2^e, m in [0.5, 1) */
  const int biased = e - 1 + 7;
  const int mant = (int)((2.0f * m - 1.0f) * 8.0f);
  return sign | (uint8_t)(biased << 3) | (uint8_t)mant;
}

ORC_API float orc_e4m3fn_decode(uint8_t b) { return e4m3fn_decode(b); }
ORC_API uint8_t orc_e4m3fn_encode(float x) { return e4m3fn_encode(x); }
ORC_API void orc_e4m3fn_encode_array(const float* in, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = e4m3fn_encode(in[i]);
}

ORC_API void orc_round_array(const float* in, float* out, int64_t n, int dtype) {
  for (int64_t i = 0; i < n; ++i) out[i] = round_to(in[i], dtype);
}

/* ------------------------------------------------------------------------ */
/* CSA                                                                        */
/* ------------------------------------------------------------------------ */

/* chunk_mean: hybrid_attention/reference.py:40-45.
 * k [B,H,S,D] -> out [B,H,S/chunk,D] fp32.  The reference requires
 * S % chunk == 0 (:41-42); this restatement covers the floor(S/chunk) complete
 * chunks, which is the same thing when the requirement holds.  Sum in double,
 * one rounding to fp32. */
ORC_API void orc_chunk_mean(const float* k, int64_t B, int64_t H, int64_t S, int64_t D,
                            int64_t chunk, float* out) {
  const int64_t C = S / chunk;
  for (int64_t bh = 0; bh < B * H; ++bh) {
    for (int64_t c = 0; c < C; ++c) {
      for (int64_t d = 0; d < D; ++d) {
        double acc = 0.0;
        for (int64_t r = 0; r < chunk; ++r) acc += (double)k[((bh * S) + c * chunk + r) * D + d];
        out[(bh * C + c) * D + d] = (float)(acc / (double)chunk);
      }
    }
  }
}

/* Order used for every top-k in this build: higher score first, and among equal
 * scores the lower chunk index first.  torch.topk (reference.py:56) leaves the
 * order of equal scores unspecified; this rule is the declared tie-break. */
static int score_before(double sa, int64_t ia, double sb, int64_t ib) {
  if (sa > sb) return 1;
  if (sa < sb) return 0;
  return ia < ib;
}

/* Partial selection sort of the first k of n (score, index) pairs. */
static void topk_sorted(const double* scores, int64_t n, int64_t k, int64_t* idx_scratch,
                        int32_t* out) {
  for (int64_t i = 0; i < n; ++i) idx_scratch[i] = i;
  for (int64_t j = 0; j < k; ++j) {
    int64_t best = j;
    for (int64_t i = j + 1; i < n; ++i) {
      const int64_t a = idx_scratch[i], b = idx_scratch[best];
      if (score_before(scores[a], a, scores[b], b)) best = i;
    }
    const int64_t t = idx_scratch[j];
    idx_scratch[j] = idx_scratch[best];
    idx_scratch[best] = t;
    out[j] = (int32_t)idx_scratch[j];
  }
}

/* select_topk_chunks scoring + selection: hybrid_attention/reference.py:48-56.
 * scores = (q . summary) * (1/sqrt(D)), top_k = min(top_k, C) (:53), sorted by
 * descending score (:56).  q [B,H,D], summary [B,H,C,D] (the chunk_mean output).
 * Writes idx [B,H,min(k,C)] and, if non-null, the double scores [B,H,C]. */
ORC_API void orc_select_topk(const float* q, const float* summary, int64_t B, int64_t H,
                             int64_t C, int64_t D, int64_t top_k, int32_t* idx,
                             double* scores_out) {
  const int64_t k = top_k < C ? top_k : C;
  const double scale = 1.0 / sqrt((double)D);
  double* sc = (double*)malloc(sizeof(double) * (size_t)(C > 0 ? C : 1));
  int64_t* scratch = (int64_t*)malloc(sizeof(int64_t) * (size_t)(C > 0 ? C : 1));
  for (int64_t bh = 0; bh < B * H; ++bh) {
    for (int64_t c = 0; c < C; ++c) {
      double acc = 0.0;
      for (int64_t d = 0; d < D; ++d)
        acc += (double)q[bh * D + d] * (double)summary[(bh * C + c) * D + d];
      sc[c] = acc * scale;
      if (scores_out) scores_out[bh * C + c] = sc[c];
    }
    if (k > 0) topk_sorted(sc, C, k, scratch, idx + bh * k);
  }
  free(sc);
  free(scratch);
}

/* Softmax attention of one query row over n gathered rows (full_decode_attention,
 * hybrid_attention/reference.py:31-37): fp32 scores scaled by 1/sqrt(D) (:34-35),
 * softmax, probabilities optionally rounded to the value dtype (:36), weighted
 * sum of value rows (:37).  rows_k/rows_v are row pointers.  out gets the
 * unrounded double result; 0 when n == 0. */
static void attend_rows(const float* q, const float* const* rows_k, const float* const* rows_v,
                        int64_t n, int64_t D, int prob_dtype, double* sc, double* out) {
  for (int64_t d = 0; d < D; ++d) out[d] = 0.0;
  if (n == 0) return;
  const double scale = 1.0 / sqrt((double)D);
  double mx = -INFINITY;
  for (int64_t t = 0; t < n; ++t) {
    double acc = 0.0;
    for (int64_t d = 0; d < D; ++d) acc += (double)q[d] * (double)rows_k[t][d];
    sc[t] = acc * scale;
    if (sc[t] > mx) mx = sc[t];
  }
  double sum = 0.0;
  for (int64_t t = 0; t < n; ++t) {
    sc[t] = exp(sc[t] - mx);
    sum += sc[t];
  }
  for (int64_t t = 0; t < n; ++t) {
    double p = sc[t] / sum;
    if (prob_dtype == ORC_BF16 || prob_dtype == ORC_F16) p = (double)round_to((float)p, prob_dtype);
    for (int64_t d = 0; d < D; ++d) out[d] += p * (double)rows_v[t][d];
  }
}

/* CSA sparse decode over explicit chunk ids.
 *   torch-csa: csa_reference -> gather_chunk_tokens -> full_decode_attention,
 *              hybrid_attention/reference.py:59-84 (prob_dtype = value dtype);
 *   cuda-csa / cuda-csa-tiled ops: csrc/csa_attention.cu:9-91,124-274, the same
 *              math with fp32 probabilities (prob_dtype = ORC_F32).
 * Slot order and edge rules follow the kernels (csa_attention.cu:46-56,170-185).
 * q [B,H,D], k/v [B,H,S,D], idx [B,H,top_k] (int64 here), out [B,H,D] double. */
ORC_API void orc_csa_attend(const float* q, const float* k, const float* v, const int64_t* idx,
                            int64_t B, int64_t H, int64_t S, int64_t D, int64_t top_k,
                            int64_t chunk, int prob_dtype, double* out, int nthreads) {
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#pragma omp parallel
#endif
  {
    const int64_t cap = top_k * chunk;
    const float** rk = (const float**)malloc(sizeof(float*) * (size_t)(cap > 0 ? cap : 1));
    const float** rv = (const float**)malloc(sizeof(float*) * (size_t)(cap > 0 ? cap : 1));
    double* sc = (double*)malloc(sizeof(double) * (size_t)(cap > 0 ? cap : 1));
#ifdef _OPENMP
#pragma omp for schedule(static)
#endif
    for (int64_t bh = 0; bh < B * H; ++bh) {
      int64_t n = 0;
      for (int64_t i = 0; i < top_k; ++i) {
        const int64_t c = idx[bh * top_k + i];
        if (c < 0) continue;
        for (int64_t off = 0; off < chunk; ++off) {
          const int64_t tok = c * chunk + off;
          if (tok >= S) break;
          rk[n] = k + (bh * S + tok) * D;
          rv[n] = v + (bh * S + tok) * D;
          ++n;
        }
      }
      attend_rows(q + bh * D, rk, rv, n, D, prob_dtype, sc, out + bh * D);
    }
    free(rk);
    free(rv);
    free(sc);
  }
  (void)nthreads;
}

/* full_decode_attention over every token: hybrid_attention/reference.py:31-37. */
ORC_API void orc_full_attend(const float* q, const float* k, const float* v, int64_t B, int64_t H,
                             int64_t S, int64_t D, int prob_dtype, double* out) {
  const float** rk = (const float**)malloc(sizeof(float*) * (size_t)(S > 0 ? S : 1));
  const float** rv = (const float**)malloc(sizeof(float*) * (size_t)(S > 0 ? S : 1));
  double* sc = (double*)malloc(sizeof(double) * (size_t)(S > 0 ? S : 1));
  for (int64_t bh = 0; bh < B * H; ++bh) {
    for (int64_t t = 0; t < S; ++t) {
      rk[t] = k + (bh * S + t) * D;
      rv[t] = v + (bh * S + t) * D;
    }
    attend_rows(q + bh * D, rk, rv, S, D, prob_dtype, sc, out + bh * D);
  }
  free(rk);
  free(rv);
  free(sc);
}

/* hca_reference: hybrid_attention/reference.py:87-92.  Chunk means of K and V
 * (fp32) cast back to the storage dtype (:90-91), then full decode attention
 * over the C summaries with probabilities rounded to that dtype (:92). */
ORC_API void orc_hca(const float* q, const float* k, const float* v, int64_t B, int64_t H,
                     int64_t S, int64_t D, int64_t chunk, int dtype, double* out) {
  const int64_t C = S / chunk;
  float* ks = (float*)malloc(sizeof(float) * (size_t)(B * H * C * D + 1));
  float* vs = (float*)malloc(sizeof(float) * (size_t)(B * H * C * D + 1));
  orc_chunk_mean(k, B, H, S, D, chunk, ks);
  orc_chunk_mean(v, B, H, S, D, chunk, vs);
  for (int64_t i = 0; i < B * H * C * D; ++i) {
    ks[i] = round_to(ks[i], dtype);
    vs[i] = round_to(vs[i], dtype);
  }
  orc_full_attend(q, ks, vs, B, H, C, D, dtype, out);
  free(ks);
  free(vs);
}

/* One CSA decode step as timed by the CPU baseline: select_topk_chunks from
 * cached fp32 summaries (reference.py:51-56 with chunk_mean hoisted out, the
 * summaries being a cache) followed by torch-csa attention over the selected
 * chunks (reference.py:69-84).  idx_scratch holds B*H*min(k,C) int64. */
ORC_API void orc_csa_decode_step(const float* q, const float* k, const float* v,
                                 const float* summary, int64_t B, int64_t H, int64_t S,
                                 int64_t D, int64_t chunk, int64_t top_k, int prob_dtype,
                                 int32_t* idx32, int64_t* idx64, double* out, int nthreads) {
  const int64_t C = S / chunk;
  const int64_t kk = top_k < C ? top_k : C;
  orc_select_topk(q, summary, B, H, C, D, kk, idx32, NULL);
  for (int64_t i = 0; i < B * H * kk; ++i) idx64[i] = idx32[i];
  orc_csa_attend(q, k, v, idx64, B, H, S, D, kk, chunk, prob_dtype, out, nthreads);
}

/* ------------------------------------------------------------------------ */
/* DSV4 paged FP8 cache                                                       */
/* ------------------------------------------------------------------------ */
/* Layout constants: hybrid_attention/dsv4_correctness.py:10-16 and
 * csrc/dsv4_attention.cu:13-19.  Per token: 448 e4m3 "nope" bytes then 64 bf16
 * "rope" values (576 bytes); after page_size such rows, page_size scale rows of
 * 8 bytes (7 UE8M0 exponents, one per 64 nope values, + 1 pad). */
#define DSV4_NOPE 448
#define DSV4_ROPE 64
#define DSV4_DIM (DSV4_NOPE + DSV4_ROPE)
#define DSV4_TILE 64
#define DSV4_SCALE_TILES (DSV4_NOPE / DSV4_TILE)
#define DSV4_ROW_BYTES (DSV4_NOPE + DSV4_ROPE * 2)
#define DSV4_SCALE_BYTES (DSV4_SCALE_TILES + 1)

/* bytes_per_page: dsv4_correctness.py:19-21. */
ORC_API int64_t orc_dsv4_bytes_per_page(int64_t page_size) {
  const int64_t raw = page_size * (DSV4_ROW_BYTES + DSV4_SCALE_BYTES);
  return ((raw + DSV4_ROW_BYTES - 1) / DSV4_ROW_BYTES) * DSV4_ROW_BYTES;
}

/* pack_dsv4_cache: dsv4_correctness.py:24-59.  k_tokens [T,512] bf16 bit
 * patterns -> cache [ceil(T/page_size), bpp] bytes (caller zero-fills). */
ORC_API void orc_dsv4_pack(const uint16_t* k_bf16, int64_t T, int64_t page_size, uint8_t* cache) {
  const int64_t bpp = orc_dsv4_bytes_per_page(page_size);
  for (int64_t loc = 0; loc < T; ++loc) {
    const int64_t page = loc / page_size, in_page = loc % page_size;
    uint8_t* pg = cache + page * bpp;
    const int64_t data_base = in_page * DSV4_ROW_BYTES;
    const int64_t scale_base = page_size * DSV4_ROW_BYTES + in_page * DSV4_SCALE_BYTES;
    const uint16_t* row = k_bf16 + loc * DSV4_DIM;
    for (int tile = 0; tile < DSV4_SCALE_TILES; ++tile) {
      float vals[DSV4_TILE];
      float max_abs = 0.0f;
      for (int j = 0; j < DSV4_TILE; ++j) {
        const uint32_t u = (uint32_t)row[tile * DSV4_TILE + j] << 16;
        memcpy(&vals[j], &u, 4);
        const float a = fabsf(vals[j]);
        if (a > max_abs) max_abs = a;
      }
      if (max_abs < 1e-8f) max_abs = 1e-8f;          /* clamp_min(1e-8) (:48) */
      const float ratio = max_abs / 448.0f;            /* fp32 tensor division (:49) */
      const double e = ceil(log2((double)ratio));      /* math.ceil(math.log2(float)) */
      const double scale = ldexp(1.0, (int)e);         /* 2.0 ** e */
      int byte = (int)e + 127;                         /* round(log2(scale)) + 127 (:50-51) */
      if (byte < 0) byte = 0;
      if (byte > 255) byte = 255;
      for (int j = 0; j < DSV4_TILE; ++j) {
        float x = vals[j] / (float)scale;              /* exact: power-of-two scale */
        if (x > 448.0f) x = 448.0f;                    /* clamp to finfo range (:52) */
        if (x < -448.0f) x = -448.0f;
        pg[data_base + tile * DSV4_TILE + j] = e4m3fn_encode(x);
      }
      pg[scale_base + tile] = (uint8_t)byte;
    }
    memcpy(pg + data_base + DSV4_NOPE, row + DSV4_NOPE, DSV4_ROPE * 2); /* raw rope (:56-57) */
  }
}

/* Dequantize one token row to 512 floats holding bf16 values:
 * dequant_dsv4_cache, dsv4_correctness.py:62-88 (nope = e4m3 * 2^(s-127) cast to
 * bf16 (:76-79,86), rope = raw bf16 (:81-83,87)); the kernel-side equivalent is
 * csrc/dsv4_attention.cu:32-56. */
static void dsv4_dequant_row(const uint8_t* cache, int64_t bpp, int64_t loc, int64_t page_size,
                             float* out) {
  const int64_t page = loc / page_size, in_page = loc % page_size;
  const uint8_t* pg = cache + page * bpp;
  const uint8_t* data = pg + in_page * DSV4_ROW_BYTES;
  const uint8_t* sc = pg + page_size * DSV4_ROW_BYTES + in_page * DSV4_SCALE_BYTES;
  for (int d = 0; d < DSV4_NOPE; ++d) {
    const float s = ldexpf(1.0f, (int)sc[d / DSV4_TILE] - 127);
    out[d] = round_bf16(e4m3fn_decode(data[d]) * s);
  }
  for (int r = 0; r < DSV4_ROPE; ++r) {
    uint16_t h;
    memcpy(&h, data + DSV4_NOPE + 2 * r, 2);
    const uint32_t u = (uint32_t)h << 16;
    memcpy(&out[DSV4_NOPE + r], &u, 4);
  }
}

ORC_API void orc_dsv4_dequant(const uint8_t* cache, int64_t bpp, const int32_t* loc, int64_t n,
                              int64_t page_size, float* out) {
  for (int64_t i = 0; i < n; ++i) dsv4_dequant_row(cache, bpp, loc[i], page_size, out + i * DSV4_DIM);
}

/* Gather the valid rows of one index list: the first clamp(length, 0, slots)
 * slots, negative entries dropped (dsv4_correctness.py:108-118,121,126-129;
 * csrc/dsv4_attention.cu:147-153,166-186).  Locations on pages beyond the cache
 * are dropped too.  Returns the row count appended at rows + n*512. */
static int64_t dsv4_gather(const uint8_t* cache, int64_t num_pages, int64_t bpp,
                           const int32_t* indices, int64_t slots, int64_t length,
                           int64_t page_size, float* rows) {
  if (length < 0) length = 0;
  if (length > slots) length = slots;
  int64_t n = 0;
  for (int64_t i = 0; i < length; ++i) {
    const int64_t loc = indices[i];
    if (loc < 0 || loc / page_size >= num_pages) continue;
    dsv4_dequant_row(cache, bpp, loc, page_size, rows + n * DSV4_DIM);
    ++n;
  }
  return n;
}

/* reference_attention: dsv4_correctness.py:91-141.  q [nq,H,512] (fp32 copy of
 * the query), SWA cache + indices [nq,T] + optional lengths [nq], optional
 * extra (C4/C128) cache + indices [nq,Te] + optional lengths, optional sink [H].
 * Per query the valid rows are shared by all heads (MQA, V = K); per head the
 * sink is a prepended logit with a zero value row (:133-137), softmax over
 * scaled scores (:133,139), out = sum p * row (:140).  out [nq,H,512] double. */
ORC_API void orc_dsv4_attention(const float* q, int64_t nq, int64_t H, const uint8_t* cache,
                                int64_t num_pages, int64_t bpp, const int32_t* indices,
                                int64_t slots, const int32_t* lengths, const float* sink,
                                int64_t page_size, double softmax_scale,
                                const uint8_t* extra_cache, int64_t extra_num_pages,
                                int64_t extra_bpp, const int32_t* extra_indices,
                                int64_t extra_slots, const int32_t* extra_lengths,
                                int64_t extra_page_size, double* out) {
  const int64_t cap = slots + (extra_cache ? extra_slots : 0);
  float* rows = (float*)malloc(sizeof(float) * (size_t)((cap > 0 ? cap : 1) * DSV4_DIM));
  double* sc = (double*)malloc(sizeof(double) * (size_t)(cap + 1));
  for (int64_t qi = 0; qi < nq; ++qi) {
    int64_t n = dsv4_gather(cache, num_pages, bpp, indices + qi * slots, slots,
                            lengths ? lengths[qi] : slots, page_size, rows);
    if (extra_cache && extra_indices && extra_slots > 0) {
      n += dsv4_gather(extra_cache, extra_num_pages, extra_bpp, extra_indices + qi * extra_slots,
                       extra_slots, extra_lengths ? extra_lengths[qi] : extra_slots,
                       extra_page_size, rows + n * DSV4_DIM);
    }
    for (int64_t h = 0; h < H; ++h) {
      const float* qv = q + (qi * H + h) * DSV4_DIM;
      double* o = out + (qi * H + h) * DSV4_DIM;
      double mx = sink ? (double)sink[h] : -INFINITY;
      for (int64_t t = 0; t < n; ++t) {
        double acc = 0.0;
        for (int d = 0; d < DSV4_DIM; ++d) acc += (double)qv[d] * (double)rows[t * DSV4_DIM + d];
        sc[t] = acc * softmax_scale;
        if (sc[t] > mx) mx = sc[t];
      }
      double sum = sink ? exp((double)sink[h] - mx) : 0.0;
      for (int64_t t = 0; t < n; ++t) {
        sc[t] = exp(sc[t] - mx);
        sum += sc[t];
      }
      for (int d = 0; d < DSV4_DIM; ++d) o[d] = 0.0;
      /* No rows: the reference's softmax/mv over an empty (or sink-only) set
       * gives zeros.  Otherwise a NaN or infinite score (a scale byte of 255
       * decodes to 2^128 = inf in fp32) makes the softmax, and so the output,
       * NaN exactly as torch.softmax does (:139-140). */
      if (n == 0) continue;
      for (int64_t t = 0; t < n; ++t) {
        const double p = sc[t] / sum;
        for (int d = 0; d < DSV4_DIM; ++d) o[d] += p * (double)rows[t * DSV4_DIM + d];
      }
    }
  }
  free(rows);
  free(sc);
}
