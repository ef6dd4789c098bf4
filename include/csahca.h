/*
 * csahca.h -- C ABI of libcsahca.so, the MI355X (gfx950) compressed-sparse-attention
 * decode library.
 *
 * This is the drop-in boundary for the CSAHCA reference's native op surface
 * (module hybrid_attention_cuda: csrc/bindings.cpp:54-163, bound from Python in
 * hybrid_attention/extension.py:13-197).  Every entry point takes plain device
 * pointers, sizes and a HIP stream, returns a status code, and never allocates:
 * scratch space comes from the caller through `workspace` (size from the
 * matching *_workspace_bytes function).  Workspace contents need no
 * initialisation, except for the decode-step entry points (csahca_csa_decode_step,
 * _dev, _at, csahca_hybrid_decode_forward's step_workspace): those keep state
 * between calls and need a zero-filled workspace (see csahca_csa_decode_step).
 * No HIP or torch type appears in a signature: `stream` is a hipStream_t passed
 * as void* (NULL = the null stream).
 *
 * Errors: a non-zero status; csahca_last_error() then returns the message of
 * the last failing call on the calling thread.  Argument errors carry the
 * reference's TORCH_CHECK texts and are detected on the host before any HIP
 * call, so they can be exercised without a GPU.
 *
 * Layouts (all row-major, contiguous):
 *   CSA:  q [batch, heads, head_dim]; k_cache, v_cache [batch, heads, seq_len,
 *         head_dim]; chunk_indices [batch, heads, top_k]; out like q;
 *         chunk summaries fp32 [batch, heads, num_chunks, head_dim].
 *   DSV4: q [num_queries, heads, 512]; caches are byte arrays [num_pages,
 *         bytes_per_page] in the DSV4 paged FP8 layout (448 e4m3 + 64 bf16 per
 *         token row, per-64 UE8M0 scale bytes after the rows of a page);
 *         token indices int32 [num_queries, slots]; lengths int32 [num_queries]
 *         or NULL; attn_sink fp32 [heads] or NULL; out like q.
 */
#ifndef CSAHCA_H_
#define CSAHCA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Storage type of q / K / V / out (the reference dispatches over f32, f64, f16
 * and bf16: AT_DISPATCH_FLOATING_TYPES_AND2, csa_attention.cu:368-383). */
enum csahca_dtype { CSAHCA_F32 = 0, CSAHCA_F16 = 1, CSAHCA_BF16 = 2, CSAHCA_F64 = 3 };

/* Chunk-index type (int32 or int64: csa_attention.cu:350-351). */
enum csahca_index_dtype { CSAHCA_I32 = 0, CSAHCA_I64 = 1 };

enum csahca_status {
  CSAHCA_OK = 0,
  CSAHCA_ERR_ARGUMENT = 1,  /* invalid argument (reference TORCH_CHECK failure) */
  CSAHCA_ERR_WORKSPACE = 2, /* workspace NULL or smaller than *_workspace_bytes */
  CSAHCA_ERR_HIP = 3        /* HIP runtime or launch error */
};

/* Message of the last failing call on this thread ("" if none). */
const char* csahca_last_error(void);

/* ABI revision of this header (bumped on incompatible changes). */
int csahca_abi_version(void);

/* ------------------------------------------------------------------------- */
/* CSA: sparse decode over explicit chunk ids                                 */
/* ------------------------------------------------------------------------- */

/* Workspace for csahca_csa_decode_forward(_tiled): fp32 split-KV partials.
 * tile_size <= 0 selects the size the untiled op uses. */
size_t csahca_csa_decode_workspace_bytes(int64_t batch, int64_t heads, int64_t head_dim,
                                         int64_t top_k, int64_t chunk_size, int64_t tile_size);

/* Replaces csa_decode_forward_cuda (csrc/csa_attention.cu:330-385; pybind op
 * csa_decode_forward, bindings.cpp:54-64).  out[b,h] = softmax over the tokens
 * of the chunks chunk_indices[b,h,:] (ids < 0 skipped, tokens >= seq_len
 * skipped) of q.k/sqrt(head_dim), applied to V; 0 when no token is valid.
 * head_dim <= 1024, chunk_size > 0. */
int csahca_csa_decode_forward(const void* q, const void* k_cache, const void* v_cache,
                              const void* chunk_indices, void* out, int dtype, int index_dtype,
                              int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                              int64_t top_k, int64_t chunk_size, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Replaces csa_decode_forward_tiled_cuda (csrc/csa_attention.cu:387-452; pybind
 * op csa_decode_forward_tiled, bindings.cpp:66-77).  Same result; tile_size (> 0)
 * is the number of selected-token slots per split-KV work item. */
int csahca_csa_decode_forward_tiled(const void* q, const void* k_cache, const void* v_cache,
                                    const void* chunk_indices, void* out, int dtype,
                                    int index_dtype, int64_t batch, int64_t heads,
                                    int64_t seq_len, int64_t head_dim, int64_t top_k,
                                    int64_t chunk_size, int64_t tile_size, void* workspace,
                                    size_t workspace_bytes, void* stream);

/* Split size the library picks for a CSA decode of this shape (>= 1). */
int64_t csahca_csa_auto_tile_size(int64_t batch, int64_t heads, int64_t top_k,
                                  int64_t chunk_size);

/* Chunk summaries: replaces chunk_mean (hybrid_attention/reference.py:40-45).
 * summary[b,h,c] = mean of rows c*chunk_size .. c*chunk_size+chunk_size-1 of
 * k_cache[b,h], in fp32, for c in [chunk_begin, chunk_begin + num_chunks).
 * Only complete chunks may be requested ((chunk_begin+num_chunks)*chunk_size
 * <= seq_len); summary holds summary_chunks >= chunk_begin+num_chunks rows per
 * head.  Recomputing one chunk is the incremental update for a growing cache. */
int csahca_csa_chunk_summary(const void* k_cache, float* summary, int dtype, int64_t batch,
                             int64_t heads, int64_t seq_len, int64_t head_dim,
                             int64_t chunk_size, int64_t summary_chunks, int64_t chunk_begin,
                             int64_t num_chunks, void* stream);

/* The incremental summary update with the token position in device memory (no
 * reference counterpart; for a decode loop captured in a HIP graph, where the
 * position advances on the device): if the token at *token_pos (int64)
 * completes chunk c = *token_pos / chunk_size ((*token_pos + 1) % chunk_size
 * == 0), summary[b,h,c] is recomputed as csahca_csa_chunk_summary does;
 * otherwise, or when chunk c lies beyond seq_len or summary_chunks, nothing is
 * written.  Summary rows thus only ever hold complete chunks. */
int csahca_csa_chunk_summary_at(const void* k_cache, float* summary, int dtype, int64_t batch,
                                int64_t heads, int64_t seq_len, int64_t head_dim,
                                int64_t chunk_size, int64_t summary_chunks,
                                const int64_t* token_pos, void* stream);

/* Workspace for csahca_csa_select_topk: the fp32 chunk scores. */
size_t csahca_csa_select_workspace_bytes(int64_t batch, int64_t heads, int64_t num_chunks);

/* Chunk selection: replaces the scoring + torch.topk of select_topk_chunks
 * (hybrid_attention/reference.py:48-56).  score[c] = (q . summary[c]) * 1/sqrt(D)
 * in fp32; out_indices[b,h,:] (int32, min(top_k, num_chunks) per head) lists the
 * best chunks by descending score, equal scores by ascending chunk id. */
int csahca_csa_select_topk(const void* q, const float* summary, int32_t* out_indices, int dtype,
                           int64_t batch, int64_t heads, int64_t num_chunks, int64_t head_dim,
                           int64_t top_k, void* workspace, size_t workspace_bytes, void* stream);

/* Workspace for csahca_csa_decode_step. */
size_t csahca_csa_step_workspace_bytes(int64_t batch, int64_t heads, int64_t num_chunks,
                                       int64_t head_dim, int64_t top_k, int64_t chunk_size);

/* One CSA decode step in a single launch (new op; it fuses select_topk_chunks,
 * hybrid_attention/reference.py:48-56 with the summaries cached, and the
 * csa_decode_forward_tiled op, csrc/csa_attention.cu:387-452): selects
 * min(top_k, num_chunks) chunks from summary [batch, heads, num_chunks,
 * head_dim] exactly as csahca_csa_select_topk (ids to out_indices), then writes
 * the sparse attention over their tokens to out, as csahca_csa_decode_forward.
 * num_chunks * chunk_size <= seq_len.  The workspace carries per-head launch
 * epochs and tagged exchange words from call to call: it must be zero-filled
 * before its first use, and zero-filled again (or replaced by another) whenever
 * (batch * heads, num_chunks, head_dim, min(top_k, num_chunks), chunk_size)
 * changes.  Every completed call leaves it reusable for the next call of the
 * same shape, including replays of a graph that captured such a call.  One
 * workspace must not be shared by calls that can run concurrently (e.g. on two
 * streams).  The workgroups of one head wait on each other, so the library
 * sizes the launch from the kernel's occupancy to be resident at once on an
 * otherwise idle device.  Should a wait still time out, the head's output is
 * NaN, csahca_csa_step_status reports it, and the head stays poisoned (NaN)
 * until the workspace is zero-filled again. */
int csahca_csa_decode_step(const void* q, const void* k_cache, const void* v_cache,
                           const float* summary, void* out, int32_t* out_indices, int dtype,
                           int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                           int64_t num_chunks, int64_t chunk_size, int64_t top_k,
                           void* workspace, size_t workspace_bytes, void* stream);

/* csahca_csa_decode_step with the chunk count in device memory (no reference
 * counterpart; for a decode loop captured in a HIP graph over a growing
 * cache): summary holds max_chunks rows per head, and the step selects among
 * the first C = clamp(*num_chunks, 0, max_chunks) of them.  out_indices holds
 * min(top_k, max_chunks) slots per head; slots past C hold -1 and add nothing
 * to the attention (C = 0 gives a zero output).  Workspace as for
 * csahca_csa_step_workspace_bytes(batch, heads, max_chunks, ...).  Needs the
 * single-launch path: float32/float16/bfloat16, head_dim 64/128/256, 16-byte
 * aligned tensors; other shapes return CSAHCA_ERR_ARGUMENT. */
int csahca_csa_decode_step_dev(const void* q, const void* k_cache, const void* v_cache,
                               const float* summary, const int32_t* num_chunks, void* out,
                               int32_t* out_indices, int dtype, int64_t batch, int64_t heads,
                               int64_t seq_len, int64_t head_dim, int64_t max_chunks,
                               int64_t chunk_size, int64_t top_k, void* workspace,
                               size_t workspace_bytes, void* stream);

/* The decode step of the token at p = *token_pos (int64, device) just
 * appended to a growing cache (no reference counterpart; for a decode loop
 * captured in a HIP graph): the chunks in play are C = min((p + 1) /
 * chunk_size, max_chunks).  If the token completes chunk C - 1 ((p + 1) a
 * multiple of chunk_size, p < seq_len), summary[b,h,C-1] is first rebuilt from
 * k_cache exactly as csahca_csa_chunk_summary computes it (same bits); then
 * the step selects among the first C rows as csahca_csa_decode_step_dev does.
 * One launch replaces csahca_csa_chunk_summary_at + csahca_csa_decode_step_dev.
 * Same workspace and shape rules as csahca_csa_decode_step_dev. */
int csahca_csa_decode_step_at(const void* q, const void* k_cache, const void* v_cache, float* summary,
                              const int64_t* token_pos, void* out, int32_t* out_indices, int dtype,
                              int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                              int64_t max_chunks, int64_t chunk_size, int64_t top_k, void* workspace,
                              size_t workspace_bytes, void* stream);

/* Reads the step workspace's sticky status word (0 = healthy; bit 0 = a
 * workgroup hand-off timed out: the affected heads returned NaN and stay
 * poisoned until the workspace is zero-filled) into host memory; synchronises
 * the stream.  workspace == NULL reads the status word of
 * csahca_csa_decode_step_noalloc's static state on the current device (no
 * reference counterpart). */
int csahca_csa_step_status(const void* workspace, uint32_t* status_out, void* stream);

/* csahca_csa_decode_step without a workspace.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation).
 * The exchange state lives in a static device array of the library (21.1 MB
 * per device, zero when the library's code object loads on that device, held
 * until the process ends); nothing is allocated and nothing needs clearing
 * between calls, whatever their shapes.  Limits: batch * heads <= 256,
 * num_chunks <= 2048, head_dim 64/128/256, float32/float16/bfloat16, 16-byte
 * aligned tensors, 0 < top_k <= 1024; other shapes return CSAHCA_ERR_ARGUMENT.
 * Results equal csahca_csa_decode_step's bit for bit.  Every call on a device
 * shares that device's array, so calls that can overlap on one device (two
 * streams) race and must be serialised by the caller.  After an exchange
 * time-out the affected head slots of the array are poisoned: every later call
 * returns NaN for the heads that use them, and the sticky status bit stays set,
 * until csahca_csa_step_noalloc_reset; csahca_csa_step_status(NULL, ...) reads
 * that status word. */
int csahca_csa_decode_step_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                   const float* summary, void* out, int32_t* out_indices, int dtype,
                                   int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                                   int64_t num_chunks, int64_t chunk_size, int64_t top_k, void* stream);

/* Zero-fills csahca_csa_decode_step_noalloc's static state on the current
 * device (status word, epochs, tagged words) with a kernel on `stream`
 * (capturable; allocates nothing).  No counterpart in the reference: it is
 * for the same callers as csahca_csa_decode_step_noalloc, to clear head slots
 * poisoned by a time-out.  Order it after every earlier and before every later
 * allocation-free call (one stream does). */
int csahca_csa_step_noalloc_reset(void* stream);

/* ------------------------------------------------------------------------- */
/* HCA: dense attention over chunk summaries, and the CSA/HCA blend           */
/* ------------------------------------------------------------------------- */

/* Workspace of csahca_hca_decode_forward: B*H*(S/chunk) fp32 scores, then
 * (256-byte aligned) B*H*(S/chunk)*head_dim fp32 V means. */
size_t csahca_hca_decode_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len,
                                         int64_t head_dim, int64_t chunk_size);

/* Replaces hca_reference (hybrid_attention/reference.py:87-92): K and V are
 * mean-pooled per chunk (fp32 mean rounded to the storage type), then full
 * decode attention over the S/chunk summary rows with probabilities rounded to
 * the storage type (reference.py:31-37).  seq_len must be a multiple of
 * chunk_size (reference.py:41-42).  With blend_src non-NULL ([B,H,D], same
 * dtype) the output is hybrid_reference's blend (reference.py:95-108):
 * round(round(w*blend) + round((1-w)*hca)), w = blend_weight. */
int csahca_hca_decode_forward(const void* q, const void* k_cache, const void* v_cache,
                              const void* blend_src, double blend_weight, void* out, int dtype,
                              int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
                              int64_t chunk_size, void* workspace, size_t workspace_bytes,
                              void* stream);

/* Replaces hybrid_reference (hybrid_attention/reference.py:95-108): the CSA
 * decode step of csahca_csa_decode_step (selection from `summary`, chunk
 * csa_chunk_size, top_k; its output to csa_out [B,H,D] and its chunk ids to
 * csa_indices [B,H,min(top_k,num_chunks)]) blended with csahca_hca_decode_forward
 * at hca_chunk_size: out = round(round(w*csa) + round((1-w)*hca)), w =
 * csa_weight.  Where the fused step runs (bf16/f16, head_dim 128, 16-byte
 * aligned tensors) the step and the HCA chunk pass share one launch, the step
 * in the first blocks; otherwise the two ops run in turn.  step_workspace
 * follows csahca_csa_decode_step's rules (zeroed once, reused, one stream);
 * hca_workspace is sized by csahca_hca_decode_workspace_bytes. */
int csahca_hybrid_decode_forward(const void* q, const void* k_cache, const void* v_cache, const float* summary,
                                 void* csa_out, int32_t* csa_indices, void* out, int dtype, int64_t batch,
                                 int64_t heads, int64_t seq_len, int64_t head_dim, int64_t num_chunks,
                                 int64_t csa_chunk_size, int64_t top_k, int64_t hca_chunk_size, double csa_weight,
                                 void* step_workspace, size_t step_workspace_bytes, void* hca_workspace,
                                 size_t hca_workspace_bytes, void* stream);

/* ------------------------------------------------------------------------- */
/* DSV4: MQA decode over the paged FP8 latent cache                           */
/* ------------------------------------------------------------------------- */

/* Workspace for the DSV4 entry points (fp32 split partials).  tile_size <= 0
 * means automatic tiling. */
size_t csahca_dsv4_decode_workspace_bytes(int64_t num_queries, int64_t heads, int64_t topk_slots,
                                          int64_t extra_topk_slots, int64_t tile_size);

/* Replaces dsv4_decode_forward_tiled_cuda (csrc/dsv4_attention.cu:762-909;
 * pybind op dsv4_decode_forward_tiled, bindings.cpp:127-155).  For query i and
 * head h: softmax over {sink[h] (value 0)} + the valid SWA slots (first
 * clamp(topk_lengths[i], 0, topk_slots), ids >= 0) + the valid extra slots, of
 * q.k * softmax_scale, applied to the dequantised rows (V = K).  extra_cache may
 * be NULL (no extra slots).  tile_size 0 = automatic.  Locations on pages at or
 * beyond num_pages are skipped. */
int csahca_dsv4_decode_forward_tiled(
    const void* q, int dtype, int64_t num_queries, int64_t heads, const uint8_t* cache,
    int64_t num_pages, int64_t bytes_per_page, int64_t page_size, const int32_t* token_indices,
    int64_t topk_slots, const int32_t* topk_lengths, const uint8_t* extra_cache,
    int64_t extra_num_pages, int64_t extra_bytes_per_page, int64_t extra_page_size,
    const int32_t* extra_token_indices, int64_t extra_topk_slots,
    const int32_t* extra_topk_lengths, const float* attn_sink, double softmax_scale,
    int64_t tile_size, void* out, void* workspace, size_t workspace_bytes, void* stream);

/* Replaces dsv4_swa_decode_forward_cuda (csrc/dsv4_attention.cu:585-657; pybind
 * op dsv4_swa_decode_forward, bindings.cpp:79-92): SWA slots only. */
int csahca_dsv4_swa_decode_forward(const void* q, int dtype, int64_t num_queries, int64_t heads,
                                   const uint8_t* cache, int64_t num_pages,
                                   int64_t bytes_per_page, int64_t page_size,
                                   const int32_t* token_indices, int64_t topk_slots,
                                   const int32_t* topk_lengths, const float* attn_sink,
                                   double softmax_scale, void* out, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* Replaces dsv4_sparse_decode_forward_cuda (csrc/dsv4_attention.cu:659-760;
 * pybind op dsv4_sparse_decode_forward, bindings.cpp:94-125): SWA + extra
 * (C4/C128) slots, extra cache required. */
int csahca_dsv4_sparse_decode_forward(
    const void* q, int dtype, int64_t num_queries, int64_t heads, const uint8_t* cache,
    int64_t num_pages, int64_t bytes_per_page, int64_t page_size, const int32_t* token_indices,
    int64_t topk_slots, const int32_t* topk_lengths, const uint8_t* extra_cache,
    int64_t extra_num_pages, int64_t extra_bytes_per_page, int64_t extra_page_size,
    const int32_t* extra_token_indices, int64_t extra_topk_slots,
    const int32_t* extra_topk_lengths, const float* attn_sink, double softmax_scale, void* out,
    void* workspace, size_t workspace_bytes, void* stream);

/* Quantize-on-write into the DSV4 cache: replaces pack_dsv4_cache
 * (hybrid_attention/dsv4_correctness.py:24-59).  k_tokens: [num_tokens, 512]
 * bf16 (16-byte aligned); token t goes to cache location locs[t] (or t when
 * locs is NULL): page loc / page_size, row loc % page_size.  Per 64-value nope
 * tile: E = ceil(log2(max(max|v|, 1e-8) / 448)), scale byte clamp(E+127, 0, 255),
 * bytes e4m3fn_rne(clamp(v / 2^E, -448, 448)); rope bf16 copied verbatim.  Writes
 * only those bytes (the reference's zero-initialised padding is the caller's).
 * Negative locations and pages at or beyond num_pages are skipped. */
int csahca_dsv4_pack_tokens(const void* k_tokens, const int32_t* locs, int64_t num_tokens, uint8_t* cache,
                            int64_t num_pages, int64_t bytes_per_page, int64_t page_size, void* stream);

/* ------------------------------------------------------------------------- */
/* Launch profiler (measurement aid; no counterpart in the reference)         */
/* ------------------------------------------------------------------------- */

/* ------------------------------------------------------------------------- */
/* Decode-block products (no reference counterpart: the reference's decode     */
/* blocks call torch's nn.Linear, hybrid_attention/model_inference.py:14-76;   */
/* these replace those calls and the elementwise ops around them in            */
/* csahca_amd.block).  W is [out_features, in_features] (nn.Linear layout),    */
/* rows of x are [batch, in_features], batch <= 4, in_features a multiple of 8 */
/* and <= 4096 (<= 2048 for batch > 1), bfloat16 or float16, x / W /           */
/* norm_weight 16-byte aligned.                                                */
/* ------------------------------------------------------------------------- */

enum csahca_activation { CSAHCA_ACT_NONE = 0, CSAHCA_ACT_SILU = 1, CSAHCA_ACT_GELU = 2 };

/* y = base + alpha * (act(x' W^T) + residual), each step rounded to the
 * storage type as the torch ops it replaces round: x' = x, or with
 * norm_weight the RMSNorm x * rsqrt(mean(x^2) + eps) * norm_weight; then the
 * product; then the activation (SiLU, or exact GELU 0.5 v (1 + erf(v/sqrt 2)));
 * then + residual if given; then base + alpha * (.) if base is given
 * (residual and base are [batch, out_features]).  y may be the same buffer as
 * residual or base (each element is read by the thread that writes it, before
 * the write) but must not overlap x.  With advance_pos, *advance_pos (int64,
 * device) is incremented by one after the product (the last kernel of a
 * decode step). */
int csahca_block_linear(const void* x, const void* norm_weight, double eps, const void* weight, int activation,
                        const void* residual, const void* base, double alpha, void* y, int dtype,
                        int64_t batch, int64_t out_features, int64_t in_features, int64_t* advance_pos,
                        void* stream);

/* The QKV projection of a decode step over a growing cache: with
 * hidden [batch, H*D], qkv = RMSNorm(hidden) w_qkv^T ([batch, 3, H, D] order)
 * goes to q [batch, H, D] and, at position p = *token_pos (int64, device), to
 * k_cache / v_cache [batch, H, capacity, D] row p (no K/V row is written when p
 * lies outside [0, capacity)); *num_chunks (int32, device, optional) is set to
 * (p + 1) / chunk_size, the complete chunks once the token is in. */
int csahca_block_qkv(const void* hidden, const void* norm_weight, double eps, const void* w_qkv, void* q,
                     void* k_cache, void* v_cache, const int64_t* token_pos, int32_t* num_chunks, int dtype,
                     int64_t batch, int64_t heads, int64_t head_dim, int64_t capacity, int64_t chunk_size,
                     void* stream);

/* Between begin and end, every kernel this thread launches through the library
 * carries a start/stop HIP event pair (hipExtLaunchKernel), which timestamps the
 * dispatch itself -- the same interval a kernel trace reports.  end waits for
 * those kernels and folds the durations per kernel name; it returns the number
 * of distinct kernels (or a negative status).  Not for use under graph capture. */
int csahca_profile_begin(void);
int csahca_profile_end(void);
int csahca_profile_result(int index, const char** kernel_name, int64_t* launches,
                          double* total_ms, double* min_ms, double* max_ms);

/* No counterpart in the reference; a timing utility for callers that capture
 * their steps into HIP graphs (bench.py times its decode steps this way).
 * csahca_device_clock_stamp launches one wavefront that stores the device wall
 * clock at *dst (device memory) when the stream reaches it; two stamps captured
 * into one graph around a run of kernels time that run on the device, without
 * the graph's launch.  csahca_device_clock_khz is that clock's rate (0 if the
 * query fails). */
int csahca_device_clock_stamp(uint64_t* dst, void* stream);
int64_t csahca_device_clock_khz(void);

#ifdef __cplusplus
}
#endif

#endif /* CSAHCA_H_ */
