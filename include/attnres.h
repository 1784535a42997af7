/*
 * attnres.h — C ABI of the MI355X (gfx950) Block Attention Residual routing
 * library, libattnres_hip.so.
 *
 * Plain pointers and sizes only: no torch or C++ types cross this boundary.
 * Every device pointer is a HIP device address on the current HIP device;
 * `stream` is a hipStream_t (NULL = the null stream).  Calls are asynchronous
 * on `stream`, allocate nothing, keep no per-call state and never synchronise.
 *
 * Return value: ATTNRES_OK (0) or a negative ATTNRES_ERR_* code;
 * attnres_last_error() then describes the failure (per thread).  Argument
 * checks run before any HIP call, so a rejected call has no device effects.
 *
 * Routing semantics, for each token row t and query q (fp32 arithmetic):
 *   qw       = query[q] * gain          (rounded to the parameter dtype)
 *   inv_rms  = rsqrt(mean_d(x_s[t]^2) + eps)
 *   logit_s  = (x_s[t] . qw) * inv_rms_s
 *   w        = softmax_s(logit)          (over the S active sources)
 *   out[q,t] = sum_s w_s * x_s[t]       (raw sources; rounded once to out dtype)
 *   lse[q,t] = max_s logit_s + log(sum_s exp(logit_s - max))
 * With S == 0 the softmax is over an empty set and every output is NaN.
 */
#ifndef ATTNRES_H
#define ATTNRES_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
#define ATTNRES_DTYPE_F32 0
#define ATTNRES_DTYPE_BF16 1

/* status codes */
#define ATTNRES_OK 0
#define ATTNRES_ERR_ARG (-1)         /* null pointer, bad size or dtype, inconsistent arguments */
#define ATTNRES_ERR_UNSUPPORTED (-2) /* shape outside what the kernels handle (S > 16, hidden) */
#define ATTNRES_ERR_ALIGN (-3)       /* pointer or row stride not 16-byte aligned */
#define ATTNRES_ERR_HIP (-4)         /* a HIP runtime call failed */

/* Largest number of active sources one routing call accepts. */
#define ATTNRES_MAX_SOURCES 16

/* Library version, major*10000 + minor*100 + patch. */
int attnres_version(void);

/* ATTNRES_MAX_SOURCES. */
int attnres_max_sources(void);

/* Message for the last failed call on this thread ("" if none). */
const char* attnres_last_error(void);

/* Kernel family used by attnres_route_fwd / attnres_block_step / attnres_merge_fwd /
 * attnres_route_bwd (process-wide). */
#define ATTNRES_POLICY_AUTO 0      /* streaming kernel for large launches, else workgroup kernel */
#define ATTNRES_POLICY_WORKGROUP 1 /* one workgroup per token row, sources held in registers */
#define ATTNRES_POLICY_STREAM 2    /* one wave per token row, sources streamed (where the shape allows) */

/*
 * Select the kernel family of routing, merge and single-query routing
 * backward calls (row per workgroup or row per wave); returns the previous
 * policy (or ATTNRES_ERR_ARG).  Both families compute the same function; AUTO
 * picks by launch size.  A tuning and testing switch with no counterpart in
 * the reference.
 */
int attnres_set_kernel_policy(int policy);

/*
 * Symbol name of the kernel a routing call launches for these arguments under
 * the current policy, for matching profiler output; written NUL-terminated
 * into buf.  fused: 0 = attnres_route_fwd (or attnres_block_step with no
 * delta and no commit), 1 = attnres_block_step or attnres_route_step
 * accumulating a delta into the partial, 2 = attnres_block_step with a
 * commit.  equally_spaced: nonzero when
 * the source pointers are equally spaced (a stacked buffer, an arena), zero
 * for arbitrary pointers (a list of separate tensors).  The same function
 * chooses the kernel here and at launch.  Loads the code object on the
 * current device.  No counterpart in the reference.
 */
int attnres_route_kernel_name(int num_sources, int64_t num_tokens, int hidden, int src_dtype, int param_dtype,
                              int out_dtype, int num_queries, int fused, int equally_spaced, char* buf,
                              int buf_len);

/*
 * Load the gfx950 code object on the current HIP device.  Optional: the
 * launch entry points call it on first use of a device.
 */
int attnres_init(void);

/*
 * One routing point: softmax over depth of S sources for num_tokens rows.
 *
 * Replaces LuxiaBaseModel._route_static (src/model/llama.py:605-644) — the
 * einsum branch llama.py:640-644 and the Triton branch llama.py:633-638 — and
 * the phase-1 op _phase_1_batched_attention_forward_with_aux
 * (src/model/flash_attn_res/ops/phase_1.py:11-66, kernel
 * kernels/phase_1.py:6-101) for num_queries >= 1.
 *
 *   sources     host array of num_sources device pointers; source s is a
 *               (num_tokens, hidden) row block with row stride src_ld elements
 *               (the reference's buf[s] for s < num_active; no stacked copy)
 *   src_dtype   ATTNRES_DTYPE_BF16 or ATTNRES_DTYPE_F32
 *   query       (num_queries, hidden), param_dtype
 *   gain        (hidden,) RMSNorm gain folded into every query, param_dtype,
 *               or NULL when `query` is already folded (phase-1 op contract)
 *   eps         RMSNorm epsilon (norm.eps)
 *   out         (num_queries, num_tokens, hidden) in out_dtype: row t of query q
 *               at out + q*out_qstride + t*out_ld elements.  out_dtype is
 *               either dtype: the einsum branch returns the promoted dtype of
 *               the sources and qw (llama.py:641-644), the phase-1 op always
 *               BF16 (ops/phase_1.py:26-30)
 *   weights     (num_queries, num_sources, num_tokens) fp32, or NULL
 *   lse         (num_queries, num_tokens) fp32, or NULL (ops/phase_1.py:32-36)
 *   inv_rms     (num_tokens, num_sources) fp32, or NULL (ops/phase_1.py:38-42)
 *   logits      (num_queries, num_tokens, num_sources) fp32, or NULL
 *               (ops/phase_1.py:44-48)
 * Requirements: 0 <= num_sources <= ATTNRES_MAX_SOURCES; hidden a multiple of
 * 8 (bf16) or 4 (fp32) and at most 8192 (bf16) / 4096 (fp32); every row start
 * 16-byte aligned.
 */
int attnres_route_fwd(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                      int64_t src_ld, int src_dtype, const void* query, const void* gain, int num_queries,
                      int param_dtype, float eps, void* out, int out_dtype, int64_t out_ld, int64_t out_qstride,
                      float* weights, float* lse, float* inv_rms, float* logits, void* stream);

/*
 * Phase-2 online-softmax merge of the intra-block partial into a phase-1
 * result (one more source joined to a softmax already taken over the
 * committed blocks):
 *   inv_rms = rsqrt(mean(p^2) + eps); logit = (p . query) * inv_rms
 *   pi = sigmoid(logit - inter_lse);   out = inter + pi * (p - inter)
 * Replaces _phase_2_online_softmax_merge_forward_with_aux
 * (src/model/flash_attn_res/ops/phase_2.py:27-71, kernel
 * kernels/phase_2.py:9-57).  `query` is pre-folded (hidden,) param_dtype;
 * partial, inter and out are contiguous (num_tokens, hidden); out has
 * inter_dtype (ops/phase_2.py:41-45); logit and inv_rms (num_tokens,) fp32 or
 * NULL.
 */
int attnres_merge_fwd(const void* partial, int64_t num_tokens, int hidden, int partial_dtype, const void* query,
                      int param_dtype, const void* inter, int inter_dtype, const float* inter_lse, float eps,
                      void* out, float* logit, float* inv_rms, void* stream);

/*
 * Symbol name of the kernel attnres_merge_fwd launches for these arguments
 * (the row-per-wave attnres_merge_stream_* or the row-per-workgroup
 * attnres_merge_*), for matching profiler output; written NUL-terminated into
 * buf (empty for num_tokens == 0, where nothing is launched).  Loads the code
 * object on the current device.  No counterpart in the reference.
 */
int attnres_merge_kernel_name(int64_t num_tokens, int hidden, int partial_dtype, int param_dtype, int inter_dtype,
                              char* buf, int buf_len);

/*
 * One routing point of the block schedule over a preallocated block arena,
 * with the partial-block update fused in.  The arena holds num_slots slots of
 * (num_tokens, hidden) rows, slot s at arena + s*slot_stride elements; slots
 * 0..n_committed-1 are committed block summaries and slot n_committed is the
 * running partial block.
 *
 *   commit == 0: partial := partial + delta (rounded to dtype; delta may be
 *                NULL for no update); route over slots 0..n_committed.
 *   commit == 1: the partial slot becomes committed block n_committed and a
 *                new partial starts in slot n_committed+1 as `delta` (required);
 *                route over slots 0..n_committed+1.
 * The updated partial is written back to its slot; `out` (num_tokens, hidden)
 * gets the routed row in `dtype`; weights/lse as in attnres_route_fwd, or NULL.
 *
 * Replaces one iteration step of the caller loops _forward_attn_res and
 * _forward_attn_res_cached (src/model/llama.py:697-715 and 742-762):
 * `_pad_and_stack` + `_route_static` + the block commit (`committed.append(
 * partial.clone()); partial = zero.clone()`) + `partial = partial + out`,
 * without the per-call stacked copy.  The caller tracks n_committed.
 */
int attnres_block_step(void* arena, int num_slots, int64_t slot_stride, int n_committed, int commit,
                       const void* delta, int64_t num_tokens, int hidden, int dtype, const void* query,
                       const void* gain, int param_dtype, float eps, void* out, float* weights, float* lse,
                       void* stream);

/*
 * One routing point of the training loop over separate block tensors, with
 * the partial-block update fused in and written to a new buffer:
 *   partial_out := partial + delta       (rounded to dtype)
 *   out         := route over committed[0 .. num_committed-1] + partial_out
 * Every row block is (num_tokens, hidden) contiguous rows of `dtype`, 16-byte
 * aligned; `partial` and `delta` are read, partial_out (which must not
 * overlap any input) and out are written; weights / lse as in
 * attnres_route_fwd, or NULL.  Unlike attnres_block_step nothing is updated in
 * place, so the partial block before the update stays valid (autograd keeps
 * it for the backward of the previous routing point).
 *
 * Replaces one iteration step of the training loop _forward_attn_res
 * (src/model/llama.py:706 or 712 `partial = partial + out`, then
 * `_pad_and_stack` + `_route_static` at 709 or 715) without the stacked copy
 * and without a separate add.
 */
int attnres_route_step(const void* const* committed, int num_committed, const void* partial, const void* delta,
                       void* partial_out, int64_t num_tokens, int hidden, int dtype, const void* query,
                       const void* gain, int param_dtype, float eps, void* out, float* weights, float* lse,
                       void* stream);

/*
 * Bytes of device workspace attnres_route_bwd and attnres_merge_bwd need for
 * num_tokens rows of `hidden` on the current device (per-workgroup fp32
 * partials of the query gradient).  An upper bound for every num_sources and
 * dtype.
 */
int attnres_route_bwd_workspace_size(int64_t num_tokens, int hidden, int64_t* bytes);

/*
 * Backward of attnres_route_fwd for one query: given dL/dout (and optionally
 * dL/dlse), writes dL/dsource for every active source and, through the fold
 * qw = query * gain, dL/dquery and dL/dgain.
 *
 * sources/src_ld/src_dtype/query/gain/param_dtype/eps: as in the forward
 * call (num_sources >= 1).  The softmax is recomputed from the sources
 * (nothing saved from the forward is needed).
 * grad_out:     (num_tokens, hidden) rows of grad_out_dtype, stride grad_out_ld.
 * grad_lse:     (num_tokens,) fp32, or NULL for no lse term.
 * grad_sources: num_sources row blocks in src_dtype, row stride grad_ld;
 *               every element of the first num_tokens rows is written.
 * workspace:    device memory of at least attnres_route_bwd_workspace_size()
 *               bytes, 16-byte aligned; its contents are scratch.
 * grad_query:   (hidden,) param_dtype, or NULL.  With gain == NULL this is
 *               dL/dqw.  grad_gain: (hidden,) param_dtype or NULL (must be
 *               NULL when gain is).  Both are written, not accumulated; the
 *               sum over tokens is taken in a fixed order (deterministic).
 *
 * Replaces the Triton backward of the phase-1 op for Q = 1
 * (src/model/flash_attn_res/ops/phase_1.py:88-284,
 * kernels/phase_1.py:104-280, kernels/reduce.py) together with the autograd of
 * `qw = query * norm.weight` (src/model/llama.py:630).  Unlike the Triton op,
 * which leaves the gradient rows of inactive slots unwritten, callers of a
 * padded buffer zero those rows themselves.
 */
int attnres_route_bwd(const void* const* sources, int num_sources, int64_t num_tokens, int hidden, int64_t src_ld,
                      int src_dtype, const void* query, const void* gain, int param_dtype, float eps,
                      const void* grad_out, int grad_out_dtype, int64_t grad_out_ld, const float* grad_lse,
                      void* const* grad_sources, int64_t grad_ld, void* workspace, int64_t workspace_bytes,
                      void* grad_query, void* grad_gain, void* stream);

/*
 * attnres_route_bwd with addend rows: grad_sources[s] = dL/dsource_s +
 * grad_addend[s], summed in fp32 and rounded once, for every s whose
 * grad_addend[s] is non-NULL (rows of grad_ld, the gradient layout).
 * grad_addend[s] may equal grad_sources[s]: the call then accumulates into
 * that gradient in place.  No two sources may share gradient or addend rows.
 * Addend rows need grad_out in the source dtype (bf16 with bf16, fp32 with
 * fp32; ATTNRES_ERR_UNSUPPORTED otherwise).  grad_addend == NULL or all-NULL
 * is attnres_route_bwd.
 *
 * Replaces autograd's summation of the gradients of a tensor that several
 * routing calls read (a committed block is a source of every later routing
 * point of the caller loop, src/model/llama.py:690-715; torch accumulates
 * each use's gradient with a separate add): with it each use's gradient is
 * added to the block's gradient inside the backward kernel.
 */
int attnres_route_bwd_add(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                          int64_t src_ld, int src_dtype, const void* query, const void* gain, int param_dtype,
                          float eps, const void* grad_out, int grad_out_dtype, int64_t grad_out_ld,
                          const float* grad_lse, void* const* grad_sources, const void* const* grad_addend,
                          int64_t grad_ld, void* workspace, int64_t workspace_bytes, void* grad_query,
                          void* grad_gain, void* stream);

/*
 * attnres_route_bwd_add for a routing point whose committed sources'
 * gradients are summed later, over every call that read them
 * (attnres_route_bwd_gather), instead of being read, added to and written
 * back at each call.  Only the gradient of the last source (the partial
 * block) is written: grad_partial = dL/dsource_{S-1} + grad_partial_addend
 * (NULL for none; may be grad_partial).  For sources s = 0 .. S-2 the call
 * stores, per token t, coef[(t*(S-1) + s)*4 + 0..3] = (w_s, c1_s, c2_s, 0)
 * (fp32; coef holds num_tokens*(S-1)*4 floats) and writes the folded query
 * query * gain (bf16, hidden values) to qfold, so that
 *   dL/dsource_s = w_s grad_out + c1_s qfold + c2_s source_s.
 * grad_query / grad_gain and the workspace as attnres_route_bwd.  Kernels
 * exist for bf16 sources, grad_out and parameters with hidden 512, 1024 or
 * 3072 (2..8 sources) or 4096 (2..9 sources); other calls return
 * ATTNRES_ERR_UNSUPPORTED and write nothing.
 *
 * Replaces, with attnres_route_bwd_gather, autograd's summation of a
 * committed block's gradient over the routing points that read it
 * (src/model/llama.py:690-715; each use's gradient is a separate tensor that
 * torch adds): the sum is formed once per block from each point's output
 * gradient and these coefficients.
 */
int attnres_route_bwd_defer(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                            int64_t src_ld, int src_dtype, const void* query, const void* gain, int param_dtype,
                            float eps, const void* grad_out, int grad_out_dtype, int64_t grad_out_ld,
                            const float* grad_lse, void* grad_partial, const void* grad_partial_addend,
                            int64_t grad_ld, float* coef, void* qfold, void* workspace, int64_t workspace_bytes,
                            void* grad_query, void* grad_gain, void* stream);

/*
 * A source's gradient summed over the num_terms calls of
 * attnres_route_bwd_defer that read it, for every token t:
 *   out = addend + sum_j (w_j grad_outs[j] + c1_j qfolds[j]) + (sum_j c2_j) x
 * with (w_j, c1_j, c2_j) = coefs[j][t*coef_lds[j] + 0..2]: for a call over
 * S_j sources that read x as source s_j, coefs[j] = its coef + 4*s_j and
 * coef_lds[j] = 4*(S_j - 1).  bf16 rows of hidden 512, 1024, 3072 or 4096 (x rows x_ld
 * apart, grad_outs[j] rows grad_out_ld, out and addend rows out_ld); addend
 * may be NULL or out (in place).  fp32 sums rounded once per group of up to
 * 48 terms (more terms: later groups add to out).  Runs the one-block
 * instance of the attnres_route_bwd_gather_seg kernels.
 *
 * See attnres_route_bwd_defer for the reference code this replaces.
 */
int attnres_route_bwd_gather(const void* x, int64_t num_tokens, int hidden, int64_t x_ld, int dtype, int num_terms,
                             const void* const* grad_outs, int64_t grad_out_ld, const float* const* coefs,
                             const int64_t* coef_lds, const void* const* qfolds, const void* addend, void* out,
                             int64_t out_ld, void* stream);

/*
 * The gradients of blocks 0 .. num_blocks-1 summed over one segment of the
 * training loop: the num_terms calls of attnres_route_bwd_defer that read
 * them all as sources 0 .. num_blocks-1 (every routing point between two
 * commits), each call's grad_out row read once for all blocks.  For every
 * token t and block k, with (w, c1, c2) = coefs[j][t*coef_lds[j] + 4*k + 0..2]
 * (coefs[j] = call j's coef, coef_lds[j] = 4*(S_j - 1) >= 4*num_blocks):
 *   sum_k  = part_in[k] + sum_j (w grad_outs[j] + c1 qfolds[j])   (bf16 rows)
 *   csum_k = csum_in[k] + sum_j c2                                (fp32)
 * Blocks k < num_blocks-1 store sum_k to part_out[k] and csum_k to
 * csum_out[k] (their running sums for the next segment); the last block, the
 * one whose commit ends the segment, stores its gradient
 *   part_out[last] = sum + csum x + addend
 * (x: its rows; addend NULL or rows of out_ld, may equal part_out[last]).
 * part_in / csum_in (the arrays or entries) may be NULL for a block's first
 * segment, or equal part_out / csum_out (in place).  More than 48 terms are
 * launched in groups, the later ones continuing from part_out / csum_out
 * (csum_out[last] is then needed as scratch).  bf16 rows of hidden 512,
 * 1024, 3072 or 4096, up to 8 blocks; other calls return
 * ATTNRES_ERR_UNSUPPORTED.
 *
 * See attnres_route_bwd_defer for the reference code this replaces.
 */
int attnres_route_bwd_gather_seg(int num_blocks, int64_t num_tokens, int hidden, int dtype, int num_terms,
                                 const void* const* grad_outs, int64_t grad_out_ld, const float* const* coefs,
                                 const int64_t* coef_lds, const void* const* qfolds, const void* const* part_in,
                                 const float* const* csum_in, void* const* part_out, float* const* csum_out,
                                 const void* x, int64_t x_ld, const void* addend, int64_t out_ld, void* stream);

/* Size of the device scratch array attnres_route_bwd_noalloc uses (32 MiB:
 * 256 CUs x 4 workgroups x 8192 fp32 columns, the largest workspace
 * attnres_route_bwd_workspace_size() reports on an MI355X). */
#define ATTNRES_NOALLOC_SCRATCH_BYTES (32u << 20)

/*
 * attnres_route_bwd without the workspace argument: the query-gradient
 * partials go to a fixed device array of ATTNRES_NOALLOC_SCRATCH_BYTES that
 * the library holds on every device it runs on until the process ends.  The
 * call allocates nothing (no hipMalloc, no allocating library routine); the
 * array's device address is resolved at set-up (attnres_init(), or the first
 * call on a device).  Under HIP graph capture, call attnres_init() on the
 * device first: a call on a capturing stream before set-up returns
 * ATTNRES_ERR_ARG.  Shapes whose workspace would exceed the array return
 * ATTNRES_ERR_UNSUPPORTED.  Every call on a device shares that device's
 * array: calls that overlap on one device (concurrent streams or threads)
 * race and must be ordered by the caller.  Results are bit-identical to
 * attnres_route_bwd with a workspace.
 *
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).
 */
int attnres_route_bwd_noalloc(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                              int64_t src_ld, int src_dtype, const void* query, const void* gain, int param_dtype,
                              float eps, const void* grad_out, int grad_out_dtype, int64_t grad_out_ld,
                              const float* grad_lse, void* const* grad_sources, int64_t grad_ld, void* grad_query,
                              void* grad_gain, void* stream);

/*
 * Symbol name of the kernel attnres_route_bwd launches for these arguments,
 * for matching profiler output; written NUL-terminated into buf.  Loads the
 * code object on the current device.  No counterpart in the reference.
 */
int attnres_route_bwd_kernel_name(int num_sources, int64_t num_tokens, int hidden, int src_dtype, int grad_out_dtype,
                                  char* buf, int buf_len);

/*
 * Bytes of device workspace attnres_route_bwd_queries needs on the current
 * device: the fp32 coefficients (num_tokens, num_queries, num_sources) plus
 * per-workgroup partials of the num_queries query gradients.
 */
int attnres_route_bwd_queries_workspace_size(int64_t num_tokens, int hidden, int num_sources, int num_queries,
                                             int64_t* bytes);

/*
 * Backward of attnres_route_fwd for num_queries >= 1 queries over the same
 * sources (the batched phase-1 call), in one pass over the sources:
 *   dL/dsource_s = sum over queries of the single-query terms,
 * plus dL/dquery for every query and dL/dgain summed over the queries.
 *
 * query:        (num_queries, hidden) param_dtype; gain (hidden,) or NULL.
 * grad_out:     num_queries blocks of (num_tokens, hidden) rows, row stride
 *               grad_out_ld, query stride grad_out_qstride (elements).
 * grad_lse:     (num_queries, num_tokens) fp32, or NULL.
 * grad_query:   (num_queries, hidden) param_dtype, or NULL; grad_gain as in
 *               attnres_route_bwd.  Sums over tokens in a fixed order.
 * workspace:    attnres_route_bwd_queries_workspace_size() bytes.
 * Other arguments as in attnres_route_bwd.  bf16 sources, output gradients
 * and parameters with num_sources <= 8, num_queries <= 8 and hidden <= 4096
 * run on the matrix cores; other shapes on the VALU kernel, which exists
 * where num_sources * 8 * V <= 72 for bf16 sources and num_sources * 4 * V
 * <= 72 for fp32 (V = 2 for rows above 512 chunks of 16 bytes).  Returns
 * ATTNRES_ERR_UNSUPPORTED for shapes neither covers; attnres_route_bwd once
 * per query covers those.
 *
 * Replaces the Triton backward of the phase-1 op for Q > 1
 * (src/model/flash_attn_res/ops/phase_1.py:88-284,
 * kernels/phase_1.py:104-280 with NUM_QUERIES_PER_BLOCK > 1, which also sums
 * the source gradients over the queries in one program), with the query
 * gradients formed in a second pass over the sources instead of per-row
 * partials (kernels/reduce.py).
 */
int attnres_route_bwd_queries(const void* const* sources, int num_sources, int64_t num_tokens, int hidden,
                              int64_t src_ld, int src_dtype, const void* query, const void* gain, int num_queries,
                              int param_dtype, float eps, const void* grad_out, int grad_out_dtype,
                              int64_t grad_out_ld, int64_t grad_out_qstride, const float* grad_lse,
                              void* const* grad_sources, int64_t grad_ld, void* workspace, int64_t workspace_bytes,
                              void* grad_query, void* grad_gain, void* stream);

/*
 * Symbol name of the first kernel attnres_route_bwd_queries launches for
 * these arguments, for matching profiler output and for tests; an empty
 * string where it would return ATTNRES_ERR_UNSUPPORTED.  Loads the code
 * object on the current device.  No counterpart in the reference.
 */
int attnres_route_bwd_queries_kernel_name(int num_sources, int hidden, int src_dtype, int param_dtype,
                                          int grad_out_dtype, int num_queries, char* buf, int buf_len);

/*
 * Backward of attnres_merge_fwd: given dL/dout (num_tokens, hidden) in
 * inter_dtype, writes dL/dpartial (partial_dtype), dL/dinter (inter_dtype),
 * dL/dinter_lse ((num_tokens,) fp32, or NULL to skip) and, when grad_query is
 * not NULL, dL/dquery ((hidden,) param_dtype, summed over tokens in a fixed
 * order).  The forward's logit and inv_rms are recomputed.  Arguments as in
 * attnres_merge_fwd; rows contiguous; workspace as for attnres_route_bwd.
 *
 * Replaces the Triton phase-2 backward
 * (src/model/flash_attn_res/ops/phase_2.py:74-255,
 * kernels/phase_2.py:60-230), whose query gradient is an fp32 atomic sum.
 */
int attnres_merge_bwd(const void* partial, int64_t num_tokens, int hidden, int partial_dtype, const void* query,
                      int param_dtype, const void* inter, int inter_dtype, const float* inter_lse, float eps,
                      const void* grad_out, void* grad_partial, void* grad_inter, float* grad_inter_lse,
                      void* workspace, int64_t workspace_bytes, void* grad_query, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ATTNRES_H */
