/*
 * Kernel-argument blocks shared by the gfx950 code object (attnres_kernels.hip)
 * and the host launcher (attnres_capi.cpp).  Both sides are compiled from this
 * one definition, so the byte layout handed to hipModuleLaunchKernel through
 * HIP_LAUNCH_PARAM_BUFFER_POINTER is the layout the kernels read.
 *
 * Plain C types only: this header is included by g++ (host) and by hipcc
 * (device) alike.
 */
#ifndef KOTODAMA_AMD_ATTNRES_PARAMS_H
#define KOTODAMA_AMD_ATTNRES_PARAMS_H

#include <stdint.h>

#define ATTNRES_KMAX_SOURCES 16   /* S templates instantiated: 0..16 */
#define ATTNRES_KMAX_WAVES 8      /* 512 threads per workgroup */

/* How the last source slot (the partial block) is formed before routing. */
#define ATTNRES_MODE_PLAIN 0      /* partial is read as-is */
#define ATTNRES_MODE_ACCUM 1      /* partial := round(partial + delta), written back */
#define ATTNRES_MODE_SET 2        /* partial := delta (fresh block after a commit), written */

/*
 * One routing point over S depth sources for n_tokens token rows.
 *   src[s]      row block of source s, token t at src[s] + t*src_ld elements
 *   query       (num_queries, d) pseudo-queries, param dtype
 *   gain        (d,) RMSNorm gain folded into every query, or NULL (pre-folded)
 *   delta       (n_tokens, d) sublayer output for MODE_ACCUM / MODE_SET, else NULL
 *   partial_out where MODE_ACCUM / MODE_SET write the updated partial rows (same row
 *               stride as the sources), or NULL to write them back over src[S-1]
 *   out         (num_queries, n_tokens, d): query q, token t at
 *               out + q*out_qstride + t*out_ld elements
 *   weights     (num_queries, S, n_tokens) fp32 softmax weights, or NULL
 *   lse         (num_queries, n_tokens) fp32 log-sum-exp of the logits, or NULL
 *   inv_rms     (n_tokens, S) fp32 rsqrt(mean(x^2)+eps), or NULL
 *   logits      (num_queries, n_tokens, S) fp32 pre-softmax logits, or NULL
 */
typedef struct attnres_route_params {
  const void* src[ATTNRES_KMAX_SOURCES];
  const void* query;
  const void* gain;
  const void* delta;
  void* partial_out;
  void* out;
  float* weights;
  float* lse;
  float* inv_rms;
  float* logits;
  int64_t n_tokens;
  int64_t src_ld;
  int64_t delta_ld;
  int64_t out_ld;
  int64_t out_qstride;
  int64_t src_stride;   /* bytes from source s to s+1 when the sources are equally spaced, else 0 */
  int32_t d;
  int32_t nchunk;       /* d / elements-per-16-byte-chunk */
  int32_t num_queries;
  int32_t param_bf16;   /* query/gain dtype: 1 bf16, 0 fp32 */
  int32_t out_bf16;     /* out dtype: 1 bf16, 0 fp32 */
  int32_t mode;         /* ATTNRES_MODE_* */
  int32_t num_sources;  /* S (the streaming kernels read it; the others are specialised on it) */
  int32_t block;        /* threads per workgroup (read as a kernel argument, not from the
                           dispatch packet, so it costs no vector load) */
  int32_t out_batch;    /* streaming kernels: finished output rows each wave stages in
                           (dynamic) LDS and stores together; 1 = store each row at once */
  float eps;
  float inv_d;
} attnres_route_params;

/*
 * Backward of one routing point (one query).  Per token, with G = grad_out:
 *   dx_s = w_s G + c1_s qw + c2_s x_s,  c1_s = dl_s r_s,  c2_s = -dl_s l_s r_s^2 / d,
 *   dl_s = w_s (G.x_s - G.out);  dqw += sum_s c1_s x_s
 * Every workgroup writes its dqw partial sum to dqw_part[blockIdx.x * d ...];
 * a reduce kernel then sums the partials in a fixed order.  The `_add`
 * kernels store dsrc[s] = dx_s + dadd[s] (rounded once) for every source with
 * a non-NULL dadd[s], which may be dsrc[s] itself (in-place accumulation).
 */
typedef struct attnres_route_bwd_params {
  const void* src[ATTNRES_KMAX_SOURCES];
  void* dsrc[ATTNRES_KMAX_SOURCES];        /* gradient rows of each source, src dtype */
  const void* dadd[ATTNRES_KMAX_SOURCES];  /* rows added to them (row stride dsrc_ld), or NULL */
  const void* query;
  const void* gain;
  const void* grad_out;  /* (n_tokens, d) */
  const float* grad_lse; /* (n_tokens,) or NULL */
  float* dqw_part;       /* (gridDim.x, d) fp32 */
  /* The `_defer` kernels: the gradients of sources 0 .. S-2 are not formed;
   * token t's coefficients of source s go to coef[(t*(S-1) + s)*4 ...] as
   * (w_s, c1_s, c2_s, 0), and workgroup 0 writes the folded query (d values,
   * param dtype) to qfold.  Only dsrc[S-1] (with dadd[S-1]) is written. */
  float* coef;
  void* qfold;
  int64_t n_tokens;
  int64_t src_ld;
  int64_t dsrc_ld;
  int64_t gout_ld;
  int32_t d;
  int32_t nchunk;
  int32_t param_bf16;
  int32_t gout_bf16;
  float eps;
  float inv_d;
} attnres_route_bwd_params;

/* One point's deferred gradient terms: its dL/dout rows, the coefficient
 * records its `_defer` backward stored and its folded query. */
typedef struct attnres_gather_term {
  const void* grad_out;  /* (n_tokens, d), row stride gout_ld */
  const float* coef;     /* token 0's (w, c1, c2, -) of the first block */
  const void* qfold;     /* (d,) */
  int64_t coef_ld;       /* floats from one token's records to the next */
} attnres_gather_term;

/*
 * One segment of the training loop's deferred gradients: the terms of the
 * points that read blocks 0 .. NB-1 (every point between two commits), summed
 * into each block's running gradient at once, so each point's dL/dout row is
 * read once however many blocks it read.  For every token t and block j:
 *   acc_j = part_in_j + sum_p (w_pj G_p + c1_pj qfold_p)      (bf16 rows)
 *   cs_j  = csum_in_j + sum_p c2_pj                           (fp32 per token)
 * with (w_pj, c1_pj, c2_pj) at term[p].coef + t*coef_ld + 4*j floats.  Blocks
 * j < NB-1 store acc_j to part_out_j and cs_j to csum_out_j; the last block
 * (the one whose commit this is) stores its gradient
 *   part_out = acc + cs x + addend.
 * part_in / csum_in may be NULL (no earlier segment) or equal part_out /
 * csum_out (in place).
 */
#define ATTNRES_SEG_MAX_BLOCKS 8
#define ATTNRES_SEG_MAX_TERMS 48
/*
 * The compiled segment kernels, attnres_route_bwd_gather_seg_c<NCH>_b<NB>:
 * X(NCH row KiB, NB blocks, CPW KiB per wave part, DEPTH ring slots, WPE waves
 * per SIMD; the host runs WPE workgroups of four waves per CU).  Shared by the
 * kernels and the host, which sizes the grid from the same parts.
 */
#ifndef ATTNRES_SEG_INSTANCES
#define ATTNRES_SEG_INSTANCES(X)                                                                        \
  X(6, 1, 3, 4, 2) X(6, 2, 3, 4, 2) X(6, 3, 3, 4, 2) X(6, 4, 3, 4, 2)                                   \
  X(6, 5, 2, 2, 2) X(6, 6, 2, 2, 2) X(6, 7, 2, 2, 2) X(6, 8, 2, 2, 2)                                   \
  X(8, 1, 4, 2, 2) X(8, 2, 4, 2, 2) X(8, 3, 4, 2, 2) X(8, 4, 4, 2, 2)                                   \
  X(8, 5, 2, 3, 2) X(8, 6, 2, 3, 2) X(8, 7, 2, 3, 2) X(8, 8, 2, 3, 2)                                   \
  X(2, 1, 2, 4, 2) X(2, 2, 2, 4, 2) X(2, 3, 2, 4, 2) X(2, 4, 2, 4, 2)                                   \
  X(2, 5, 2, 2, 2) X(2, 6, 2, 2, 2) X(2, 7, 2, 2, 2) X(2, 8, 2, 2, 2)                                   \
  X(1, 1, 1, 8, 2) X(1, 2, 1, 8, 2) X(1, 3, 1, 8, 2) X(1, 4, 1, 8, 2)                                   \
  X(1, 5, 1, 8, 2) X(1, 6, 1, 8, 2) X(1, 7, 1, 8, 2) X(1, 8, 1, 8, 2)
#endif
typedef struct attnres_seg_block {
  const void* part_in;   /* (n_tokens, d), row stride out_ld, or NULL */
  const float* csum_in;  /* (n_tokens,), or NULL */
  void* part_out;        /* (n_tokens, d), row stride out_ld */
  float* csum_out;       /* (n_tokens,); unused for the last block */
} attnres_seg_block;

typedef struct attnres_route_bwd_gather_seg_params {
  const void* x;       /* (n_tokens, d) rows of the last block, stride x_ld */
  const void* addend;  /* (n_tokens, d), stride out_ld, or NULL: added to the last block's gradient */
  int64_t n_tokens;
  int64_t x_ld;
  int64_t gout_ld;
  int64_t out_ld;
  int32_t d;
  int32_t num_terms;   /* 0 .. ATTNRES_SEG_MAX_TERMS */
  int32_t block;       /* threads per workgroup */
  int32_t final_block; /* 1: the last block takes x and the addend and stores its gradient;
                          0: it is stored like the others (running sum + csum_out) */
  attnres_gather_term term[ATTNRES_SEG_MAX_TERMS];
  attnres_seg_block blk[ATTNRES_SEG_MAX_BLOCKS];
} attnres_route_bwd_gather_seg_params;

/*
 * Backward of Q >= 2 queries over one set of sources (the batched phase-1
 * call), source gradients in one pass:
 *   dx_s = sum_q (w_qs G_q + c1_qs qw_q) + (sum_q c2_qs) x_s
 * with c1_qs stored to `c1` (n_tokens, Q, S) for the query gradients.
 */
typedef struct attnres_route_bwd_mq_params {
  const void* src[ATTNRES_KMAX_SOURCES];
  void* dsrc[ATTNRES_KMAX_SOURCES];
  const void* query;     /* (Q, d) param dtype */
  const void* gain;      /* (d,) param dtype, or NULL */
  const void* grad_out;  /* (Q, n_tokens) rows of gout_ld, query stride gout_qstride */
  const float* grad_lse; /* (Q, n_tokens) or NULL */
  float* c1;             /* (n_tokens, Q, S) fp32 */
  int64_t n_tokens;
  int64_t src_ld;
  int64_t dsrc_ld;
  int64_t gout_ld;
  int64_t gout_qstride;
  int32_t d;
  int32_t nchunk;
  int32_t num_queries;
  int32_t param_bf16;
  int32_t block;
  float eps;
  float inv_d;
} attnres_route_bwd_mq_params;

/*
 * Query-gradient partials of the batched backward: per workgroup
 *   part[wg][q][:] = sum over its rows, sources of c1_qs x_s
 * for queries q0 .. q0+7 (one more pass over the sources).
 */
typedef struct attnres_route_bwd_dqw_params {
  const void* src[ATTNRES_KMAX_SOURCES];
  const float* c1;  /* (n_tokens, Q, S) */
  float* part;      /* (gridDim.x, Q, d) */
  int64_t n_tokens;
  int64_t src_ld;
  int32_t d;
  int32_t nchunk;
  int32_t num_sources;
  int32_t num_queries;
  int32_t q0;
  int32_t block;
} attnres_route_bwd_dqw_params;

/* Column reduction of the dqw partials into the parameter gradients. */
typedef struct attnres_reduce_params {
  float* part;        /* (nparts, num_queries * d); stage 1 overwrites rows 0, 64, 128, ... */
  const void* query;  /* (num_queries, d) param dtype */
  const void* gain;   /* (d,) param dtype, or NULL */
  void* dquery;       /* (num_queries, d) param dtype: dqw * gain (dqw when gain is NULL) */
  void* dgain;        /* (d,) param dtype: sum over queries of dqw * query, or NULL */
  int32_t nparts;     /* rows of `part` written by the backward kernel */
  int32_t part_step;  /* final stage sums rows 0, part_step, 2*part_step, ... */
  int32_t d;
  int32_t param_bf16;
  int32_t num_queries; /* 0 or 1: one query */
} attnres_reduce_params;

/*
 * Online-softmax merge of one intra-block partial into a phase-1 result:
 *   inv_rms = rsqrt(mean(p^2)+eps); logit = (p . q) * inv_rms
 *   pi = sigmoid(logit - inter_lse); out = inter + pi * (p - inter)
 */
typedef struct attnres_merge_params {
  const void* partial;    /* (n_tokens, d), partial dtype */
  const void* query;      /* (d,) pre-folded, param dtype */
  const void* inter;      /* (n_tokens, d), inter dtype */
  const float* inter_lse; /* (n_tokens,) */
  void* out;              /* (n_tokens, d), inter dtype */
  float* logit;           /* (n_tokens,) or NULL */
  float* inv_rms;         /* (n_tokens,) or NULL */
  int64_t n_tokens;
  int64_t partial_ld;
  int64_t inter_ld;
  int64_t out_ld;
  int32_t d;
  int32_t nchunk;
  int32_t param_bf16;
  int32_t inter_bf16;
  int32_t block;          /* threads per workgroup */
  float eps;
  float inv_d;
} attnres_merge_params;

/* Phase-2 merge backward. */
typedef struct attnres_merge_bwd_params {
  const void* partial;    /* (n_tokens, d), partial dtype */
  const void* query;      /* (d,) pre-folded, param dtype */
  const void* inter;      /* (n_tokens, d), inter dtype */
  const float* inter_lse; /* (n_tokens,) */
  const void* grad_out;   /* (n_tokens, d), inter dtype */
  void* grad_partial;     /* (n_tokens, d), partial dtype */
  void* grad_inter;       /* (n_tokens, d), inter dtype */
  float* grad_lse;        /* (n_tokens,) or NULL */
  float* dq_part;         /* (gridDim.x, d) fp32 */
  int64_t n_tokens;
  int32_t d;
  int32_t nchunk;
  int32_t param_bf16;
  float eps;
  float inv_d;
} attnres_merge_bwd_params;

#endif /* KOTODAMA_AMD_ATTNRES_PARAMS_H */
