/*
 * triton_llm_hip.h -- C ABI of libtriton_llm_hip.so, the gfx950 (MI355X)
 * attention path behind triton_llm's Python entry points.
 *
 * Every function returns an int status: 0 on success, otherwise a hipError_t
 * value (argument errors use TL_ERR_INVALID = hipErrorInvalidValue, shapes the
 * kernels do not cover use TL_ERR_UNSUPPORTED = hipErrorNotSupported).
 * tl_error_string() turns a status into text.
 *
 * Conventions
 *   - Pointers are device pointers unless named host_*.
 *   - Strides are in ELEMENTS, as in the reference kernels
 *     (triton_llm/kernels/attention.py:48-49 "Row strides in elements").
 *     The head dimension is always contiguous (stride 1).
 *   - `stream` NULL means the library's own stream (created by tl_init);
 *     all launches and copies the Python layer issues go to that stream, so
 *     stream order replaces the reference's per-call device synchronize.
 *   - The library never allocates device memory on its own.  Scratch
 *     ("workspace") is passed in by the caller, sized by the *_workspace_bytes
 *     query functions.
 *   - dtype codes: TL_DTYPE_F32, TL_DTYPE_F16, TL_DTYPE_BF16.  Softmax and
 *     accumulation always run in fp32.
 */
#ifndef TRITON_LLM_HIP_H
#define TRITON_LLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TL_DTYPE_F32 0
#define TL_DTYPE_F16 1
#define TL_DTYPE_BF16 2

#define TL_ERR_INVALID 1       /* hipErrorInvalidValue */
#define TL_ERR_UNSUPPORTED 801 /* hipErrorNotSupported */

/* ---------------------------------------------------------------------------
 * Runtime / allocator.  Replaces the ctypes bindings the reference's
 * triton_llm/gpu.py makes directly on libamdhip64 / libcudart:
 *   hipMalloc      gpu.py:120-121, :230-236   -> tl_malloc
 *   hipFree        gpu.py:123-124, :194-200   -> tl_free
 *   hipMemcpy H2D  gpu.py:215-224             -> tl_memcpy_htod (async on the
 *                                                library stream + stream sync)
 *   hipMemcpy D2H  gpu.py:202-213             -> tl_memcpy_dtoh (idem)
 *   hipDeviceSynchronize gpu.py:252-263       -> tl_synchronize
 *   backend probe  gpu.py:47-86               -> tl_device_count / tl_init
 * ------------------------------------------------------------------------- */
int tl_device_count(int* count);
int tl_init(int device);
void* tl_default_stream(void);
int tl_malloc(void** ptr, size_t nbytes);
int tl_free(void* ptr);
int tl_memcpy_htod(void* dst, const void* host_src, size_t nbytes);
int tl_memcpy_dtoh(void* host_dst, const void* src, size_t nbytes);
int tl_memcpy_dtod(void* dst, const void* src, size_t nbytes);
int tl_memset(void* dst, int value, size_t nbytes);
int tl_synchronize(void);
const char* tl_error_string(int status);

/* Event timing (no counterpart in the reference, which times nothing below
 * the Python wall clock; used by bench.py for per-kernel durations). */
int tl_event_create(void** event);
int tl_event_destroy(void* event);
int tl_event_record(void* event, void* stream);
int tl_event_synchronize(void* event);
int tl_event_elapsed_ms(float* ms, void* start, void* stop);

/* HIP graphs of a sequence of calls (no counterpart in the reference, whose
 * every call goes through the Python launcher).  tl_graph_capture_begin
 * starts recording `stream` (NULL: the library stream); every tl_* launch
 * and device-to-device copy issued to it until tl_graph_capture_end is
 * recorded, not run.  Calls that synchronise (tl_memcpy_htod / _dtoh,
 * tl_synchronize) must not be issued while recording; tl_memset (a fill
 * kernel on the library stream) may.
 * tl_graph_capture_end returns an executable graph; tl_graph_launch replays
 * it on a stream with the pointers and sizes it was recorded with.  A
 * decode step of a serving loop is a few small kernels whose host launch
 * cost exceeds their run time: replaying it as one graph keeps the GPU busy. */
int tl_graph_capture_begin(void* stream);
int tl_graph_capture_end(void* stream, void** exec);
int tl_graph_launch(void* exec, void* stream);
int tl_graph_destroy(void* exec);

/* ---------------------------------------------------------------------------
 * RoPE, in place.  Replaces apply_rope (triton_llm/kernels/rope.py:153-222)
 * and its _rope_kernel (rope.py:25-70): half-split pairing (i, i + d_k/2),
 * position = (row % seq_len) + position_offset, cos/sin tables half-packed
 * fp32 (max_seq, d_k/2).  The rotation is evaluated as separately rounded
 * fp32 multiplies and adds (no FMA contraction) and rounded once to the
 * storage type, so results are bit-identical to the NumPy restatement.
 * ------------------------------------------------------------------------- */
int tl_rope_inplace(void* x, const float* cos_table, const float* sin_table,
                    int64_t n_rows, int64_t row_stride, int d_k, int seq_len,
                    int position_offset, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Attention forward (prefill / general Sq x Sk).  Replaces
 *   attention_gqa + _gqa_attention_kernel (attention_gqa.py:149-269, :21-146)
 *   attention     + _attention_kernel     (attention.py:141-216, :18-138)
 * Q: (batch, n_head, seq_q, d_k), K/V: (batch, n_kv_head, seq_k, d_k), O like Q,
 * each given by {batch, head, seq} element strides.  Query head h reads KV head
 * h / (n_head / n_kv_head) (attention_gqa.py:76).  causal != 0 masks key j for
 * query i when j > i + (seq_k - seq_q) (bottom-right alignment,
 * attention_gqa.py:97; equal to attention.py's top-left mask when
 * seq_q == seq_k).  Scores are (q . k) * sm_scale.
 * Requires seq_q >= 1, seq_k >= 1 (the Python layer returns the reference's
 * empty/zero results itself).  d_k 64 and 128 with 16-byte-aligned rows run
 * the MFMA kernels; any other d_k up to 4096 (the reference accepts any
 * power of two) runs a generic fp32 kernel; larger d_k returns
 * TL_ERR_UNSUPPORTED.  fp16 with |sm_scale| * log2(e) > 1 scales the scores
 * in fp32 instead of pre-scaling Q, whose fp16 copy could overflow.
 * Workspace: tl_attention_fwd_workspace_bytes
 * (the 16-bit MFMA path at d_k 128 stages a key-major copy of V there; 0
 * for d_k 64 and fp32, which read V in place; NULL is accepted when 0).
 * A 16-byte-aligned workspace of tl_attention_fwd_workspace_bytes_split
 * bytes (at least the above) also lets a causal 16-bit MFMA call with
 * seq_k >= seq_q and few query tiles split the key range of its costliest
 * tiles over two workgroups, which balances the persistent schedule; the
 * two parts of a tile merge inside the kernel (no extra launch).  Given
 * less, the call runs unsplit.  Split and unsplit outputs agree to rounding;
 * either is deterministic for the same arguments and workspace size.  The
 * workspace needs no initialisation and may be reused by later calls (on
 * one stream, as the V copy requires).
 * ------------------------------------------------------------------------- */
size_t tl_attention_fwd_workspace_bytes(int batch, int n_kv_head, int seq_k,
                                        int d_k, int dtype);
/* No counterpart in the reference (its attention launches take no
 * workspace); see above. */
size_t tl_attention_fwd_workspace_bytes_split(int batch, int n_head, int n_kv_head,
                                              int seq_q, int seq_k, int d_k,
                                              int causal, int dtype);
int tl_attention_fwd(const void* q, const void* k, const void* v, void* o,
                     void* workspace, size_t workspace_bytes, int batch,
                     int n_head, int n_kv_head, int seq_q, int seq_k, int d_k,
                     const int64_t* q_strides, const int64_t* k_strides,
                     const int64_t* v_strides, const int64_t* o_strides,
                     float sm_scale, int causal, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Single-token decode over a preallocated KV cache (split-K + log-sum-exp
 * combine).  The reference does this with attention_gqa(q, K[:L], V[:L],
 * causal=False) after re-uploading the cache prefix every step
 * (smollm2_triton/model.py:299-314; gpt2_triton/model.py:332-349); here the
 * cache stays resident and is read in place.
 * Q/O: (batch, n_head, d_k) with {batch, head} strides.  Caches:
 * (batch, n_kv_head, max_ctx, d_k) with {batch, head, seq} strides.
 * Sequence b attends to positions [0, min(cache_lens[b] + len_add, max_ctx)).
 * cache_lens may be NULL: every sequence then attends to len_add positions
 * (a caller that knows the length on the host passes it by value, with no
 * upload).
 * The cached positions of all sequences and KV heads are cut into equal
 * shares, one per resident workgroup of the device; split_size (multiple of
 * 16; 0 picks tl_decode_split_size) is the smallest share, which bounds the
 * partials one (sequence, head) can produce: ceil(max_ctx / split_size) + 1.
 * Launches the split pass, then a combine pass that merges the partials of
 * heads whose positions were shared by several workgroups and writes zeros
 * for empty sequences.  The workspace holds the partials and may be reused
 * by consecutive calls on one stream.  Small caches (max_ctx <= 2048, at
 * most 384 KiB of K and V per (sequence, KV head) at max_ctx and 64 MiB in
 * all) instead run one workgroup per (sequence, KV head)
 * that finishes its heads itself: one launch, no partials, and the kernels
 * read neither split_size nor the workspace.  The workspace arguments are
 * checked in every mode all the same (non-NULL, 16-byte aligned, at least
 * tl_attention_decode_workspace_bytes), so a caller never depends on which
 * mode a shape takes.  (TRITON_LLM_HIP_DECODE_SHARES=1 in the environment
 * when tl_init runs forces the shares path; tests use it.)
 * d_k is 64 or 128.  Each lane reads a slice of d_k / 16 elements of a
 * row (d_k / 8 for 16-bit d_k 64 in the small-cache mode with at most 4
 * query heads per KV head), so q, k_cache, v_cache and every q / k / v
 * stride must be multiples of that slice; otherwise, or when one (sequence,
 * head) region of a cache exceeds 2 GiB, the call returns
 * TL_ERR_UNSUPPORTED.
 * ------------------------------------------------------------------------- */
int tl_decode_split_size(int batch, int n_kv_head, int max_ctx);
size_t tl_attention_decode_workspace_bytes(int batch, int n_head, int max_ctx,
                                           int d_k, int split_size);
int tl_attention_decode(const void* q, const void* k_cache, const void* v_cache,
                        const int32_t* cache_lens, int len_add, void* o,
                        void* workspace, size_t workspace_bytes, int batch,
                        int n_head, int n_kv_head, int max_ctx, int d_k,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides,
                        float sm_scale, int split_size, int dtype,
                        void* stream);

/* One decode step's token and attention in one call:
 *   tl_rope_kv_append(q, k_new, v_new, ..., n_new = 1)  then
 *   tl_attention_decode(q, k_cache, v_cache, cache_lens, len_add = 1, ...)
 * with the same results (rotated q in place, cache row cache_lens[b]
 * written bit for bit as tl_rope_kv_append writes it, the same output).
 * No reference counterpart as one function: it fuses the model's decode
 * sequence (smollm2_triton/model.py:296-314; gpt2_triton/model.py:332-349
 * without RoPE).  In the small-cache mode the workgroup of each (sequence,
 * KV head) rotates and writes its token before streaming the cache, so the
 * step is one launch; otherwise the append is its own launch first.
 * q: (batch, n_head, d_k) {batch, head} strides, rotated in place;
 * k_new / v_new: (batch, n_kv_head, d_k) {batch, head} strides, read only;
 * caches, o, workspace, split_size and the support rules as for
 * tl_attention_decode; cos/sin (rope_rows rows of d_k / 2) as for
 * tl_rope_kv_append (NULL: no RoPE).  cache_lens must not be NULL. */
int tl_attention_decode_append(void* q, const void* k_new, const void* v_new,
                               void* k_cache, void* v_cache, const int32_t* cache_lens,
                               const float* cos_table, const float* sin_table,
                               int rope_rows, void* o, void* workspace,
                               size_t workspace_bytes, int batch, int n_head,
                               int n_kv_head, int max_ctx, int d_k,
                               const int64_t* q_strides, const int64_t* k_new_strides,
                               const int64_t* v_new_strides, const int64_t* k_strides,
                               const int64_t* v_strides, const int64_t* o_strides,
                               float sm_scale, int split_size, int dtype, void* stream);

/* The same decode with no workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  The
 * split partials live in a static device array of
 * TL_DECODE_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends;
 * problems whose tl_attention_decode_workspace_bytes exceeds it return
 * TL_ERR_INVALID before any device work.  No hipMalloc / hipFree or other
 * allocating call is made.  Calls that overlap in time on one GPU share that
 * array and race: issue them on one stream.  Results are identical to
 * tl_attention_decode's for the same arguments. */
#define TL_DECODE_NOALLOC_SCRATCH_BYTES (32u << 20)
/* The same limit as a data symbol of the loaded library, so a binding reads
 * it from the library it calls instead of repeating the number. */
extern const size_t tl_decode_noalloc_scratch_bytes;
int tl_attention_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                const int32_t* cache_lens, int len_add, void* o, int batch,
                                int n_head, int n_kv_head, int max_ctx, int d_k,
                                const int64_t* q_strides, const int64_t* k_strides,
                                const int64_t* v_strides, const int64_t* o_strides,
                                float sm_scale, int split_size, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * RoPE + KV-cache append, fused into the Q/K write.  Replaces the model's
 * host-side sequence  apply_rope(q) ; apply_rope(k) ; k/v -> host ;
 * cache[:, len] = k/v  (smollm2_triton/model.py:296-308 decode,
 * :332-339 prefill; gpt2_triton/model.py:339-341 without RoPE).
 * q: (batch, n_new, n_head, d_k) rotated in place (may be NULL);
 * k_new / v_new: (batch, n_new, n_kv_head, d_k), read only;
 * token s of sequence b is written to cache position cache_lens[b] + s, after
 * RoPE at that position for q and k.  cos/sin NULL disables RoPE (GPT-2).
 * Positions >= max_ctx (or >= rope_rows when RoPE is on) are not written.
 * Strides: q/k_new/v_new {batch, seq, head}; caches {batch, head, seq}.
 * ------------------------------------------------------------------------- */
int tl_rope_kv_append(void* q, const void* k_new, const void* v_new,
                      void* k_cache, void* v_cache, const int32_t* cache_lens,
                      const float* cos_table, const float* sin_table,
                      int rope_rows, int batch, int n_new, int n_head,
                      int n_kv_head, int max_ctx, int d_k,
                      const int64_t* q_strides, const int64_t* k_new_strides,
                      const int64_t* v_new_strides,
                      const int64_t* k_cache_strides,
                      const int64_t* v_cache_strides, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Dense projection GEMM of the model step: C = A . B, row-major, A (m, k) with row stride lda, B
 * (k, n) with ldb, C (m, n) with ldc, all of one dtype, fp32 accumulation.
 * Replaces the Triton GEMM gemm(h_dev, w_dev, out_dev)
 * (triton_llm/kernels/gemm.py:53-108) used for every projection in
 * gpt2_triton/model.py and smollm2_triton/model.py (e.g. :285-287, :351,
 * :360-363, :375).  k = 0 writes zeros; m = 0 or n = 0 does nothing.
 * m <= 8 (a decoded token) runs a hand-written HBM-streaming kernel whose
 * K-slice partial sums need tl_gemm_workspace_bytes(m, n, k, dtype) bytes of
 * workspace; larger m runs a hand-written MFMA kernel (128 x 128 tiles of
 * C, or 256 x 256 for large 16-bit products; rows of A and B must be
 * 16-byte aligned, otherwise a simple FMA kernel takes the product), which
 * for fp32 products that leave CUs unevenly loaded, and for products of
 * any dtype with fewer than two tiles per CU (a batch of decoded tokens:
 * at most 64 rows take 64 x 128 tiles), splits K and keeps fp32 partials in
 * the workspace.  The query gives 0 when no workspace is used.
 * Given less than the query asks for, the MFMA kernel runs whole-K instead
 * of failing; the skinny kernel needs its workspace.
 * ------------------------------------------------------------------------- */
size_t tl_gemm_workspace_bytes(int m, int n, int k, int dtype);
int tl_gemm(const void* a, const void* b, void* c, int m, int n, int k, int64_t lda,
            int64_t ldb, int64_t ldc, void* workspace, size_t workspace_bytes, int dtype,
            void* stream);
/* Up to four products that share A, C_g = A . B_g with B_g (k, n[g]),
 * in one launch (plus one split-K reduce launch for all of them when K is
 * split):
 * the q/k/v projections of a layer, or gate/up.  No reference counterpart as
 * one call: the reference's model calls gemm (gemm.py:53-108) once per
 * projection (smollm2_triton/model.py:285-287, :360-361).  Per group the
 * arguments mean what tl_gemm's mean; groups with n[g] = 0 are skipped.
 * Workspace: tl_gemm_grouped_workspace_bytes(m, k, count, n, dtype). */
size_t tl_gemm_grouped_workspace_bytes(int m, int k, int count, const int* n, int dtype);
int tl_gemm_grouped(const void* a, int m, int k, int64_t lda, int count,
                    const void* const* b, void* const* c, const int* n,
                    const int64_t* ldb, const int64_t* ldc, void* workspace,
                    size_t workspace_bytes, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Layers around the projections, contiguous rows, fp32 math in any dtype.
 *   tl_rms_norm: y = (x / sqrt(mean(x^2) + eps)) * w per row of n; replaces
 *     rms_norm(x_dev, w_dev, out_dev, eps) (triton_llm/kernels/rms_norm.py:68-116).
 *   tl_add_rms_norm: h = a + b, then y = rms_norm(h) (the residual add and
 *     the next RMSNorm of smollm2_triton/model.py:352-357 / :279-280 in one
 *     pass; h is written, and normalised as stored).  No reference
 *     counterpart as one call: it fuses add.py:54-104 with rms_norm.py.
 *   tl_swiglu: out = silu(gate) * up, count elements; replaces
 *     swiglu(gate_dev, up_dev, out_dev) (triton_llm/kernels/swiglu.py:70-125).
 *   tl_add: z = x + y, count elements; replaces add(x_dev, y_dev, out_dev)
 *     (triton_llm/kernels/add.py:54-104).
 * m = 0 or count = 0 does nothing; n = 0 rows are an error, as in rms_norm.py:96-97.
 * ------------------------------------------------------------------------- */
int tl_rms_norm(const void* x, const void* w, void* y, int m, int n, float eps, int dtype,
                void* stream);
int tl_add_rms_norm(const void* a, const void* b, void* h, const void* w, void* y, int m,
                    int n, float eps, int dtype, void* stream);
int tl_swiglu(const void* gate, const void* up, void* out, int64_t count, int dtype,
              void* stream);
int tl_add(const void* x, const void* y, void* z, int64_t count, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Next-token sampling, one token per row of logits [rows][row_stride]
 * (vocab valid entries per row); replaces SmolLM2._sample
 * (smollm2_triton/model.py:566-584; GPT-2: gpt2_triton/model.py:424-438),
 * which runs on the host after downloading the logits.
 *   temperature <= 0: tokens[r] = first index of the row's maximum (np.argmax;
 *     a NaN counts as the maximum).  uniforms may be NULL.
 *   temperature > 0: p = exp(x / T - max / T); 0 < top_k < vocab keeps every
 *     entry >= the top_k-th largest logit (ties with it all kept); tokens[r] =
 *     first index whose cumulative kept mass exceeds uniforms[r] * total, the
 *     inverse CDF np.random.choice applies to its uniform draw.  A row whose
 *     maximum is not finite (NaN / +inf logits, all -inf) gets -1, where the
 *     reference's np.random.choice raises ValueError.
 * The reference's 1e-6 greedy cut-off is the caller's (compare in double,
 * pass 0 for greedy).  1 <= vocab <= tl_sample_max_vocab(), row_stride >=
 * vocab, top_k >= 0 (0 keeps all), rows <= 65535; rows = 0 does nothing.
 * workspace: tl_sample_workspace_bytes(rows, vocab) bytes (segment results
 * and candidates; no initial contents needed).  Two kernels on `stream`:
 * one workgroup per 2048-entry segment of every row, then one per row.
 * ------------------------------------------------------------------------- */
int tl_sample_max_vocab(void);
size_t tl_sample_workspace_bytes(int rows, int vocab);
int tl_sample(const void* logits, int rows, int vocab, int64_t row_stride, float temperature,
              int top_k, const double* uniforms, int32_t* tokens, void* workspace,
              size_t workspace_bytes, int dtype, void* stream);
/* One row, the draw passed by value: the per-token call of the models'
 * generate loops (smollm2_triton/model.py:458-460), with no draw upload.
 * Same results as tl_sample with rows = 1 and uniforms = {uniform};
 * workspace: tl_sample_workspace_bytes(1, vocab). */
int tl_sample_row(const void* logits, int vocab, float temperature, int top_k, double uniform,
                  int32_t* token, void* workspace, size_t workspace_bytes, int dtype,
                  void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRITON_LLM_HIP_H */
