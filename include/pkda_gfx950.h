/*
 * pkda_gfx950.h -- C ABI of the MI355X (gfx950) PKDA recurrence library.
 *
 * PKDA is the preconditioned Kimi-delta-attention recurrence of
 * a9lim/delta-feedback-experiment.  Per head, with FP32 state S [K x V] and
 * FP32 preconditioner state A [K]:
 *
 *   A_t  = exp(g_atk_t) A_{t-1} + beta_atk_t (k_t * k_t)
 *   kw_t = k_t * exp(-ln(x) r_t / (1 + |r_t|)),   r_t = log(A_t + eps) - center
 *   S'   = diag(exp(g_t)) S_{t-1}
 *   S_t  = S' + beta_t kw_t (v_t - S'^T k_t)^T
 *   o_t  = S_t^T (scale q_t)
 *
 * (reference: delta_feedback_experiment/pkda.py:355-410).
 *
 * Conventions shared by every entry point:
 *  - Pointers are device pointers; every tensor is dense row-major in the
 *    shape its comment gives.  Token tensors are "flat": [N_tok, H, D] where
 *    N_tok = batch * seqlen for equal-length rows, or the packed length when
 *    cu_seqlens (int32 [num_seqs + 1], device) is given.
 *  - dk == dv == D, and D is one of 64 or 128 (32 for the token-recurrent
 *    and decode kernels as well).
 *  - `stream` is a hipStream_t passed as void*.  Calls only enqueue work: the
 *    library never allocates or frees device memory, never synchronises the
 *    host and keeps no state besides the last error message (and the static
 *    device array of pkda_gate_bwd_noalloc), so a caller may capture every
 *    call into a HIP graph.
 *  - Return value: 0 on success; < 0 for an argument rejected before any
 *    launch (PKDA_E*); > 0 is the hipError_t of a failed launch.  The
 *    message of the last failure on the calling thread is pkda_last_error().
 *  - Outputs are deterministic: no floating-point atomics anywhere.
 */
#ifndef PKDA_GFX950_H
#define PKDA_GFX950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKDA_ABI_VERSION 13
#define PKDA_CHUNK 64

enum pkda_dtype { PKDA_F32 = 0, PKDA_BF16 = 1 };

enum pkda_status {
  PKDA_OK = 0,
  PKDA_EINVAL = -1,       /* null pointer, bad size, struct_size mismatch */
  PKDA_EUNSUPPORTED = -2, /* head dim / dtype / combination not built */
  PKDA_ERANGE = -3        /* an index out of range (checked on the host only when stated) */
};

/* Gate forms.  All decays are natural-log, <= 0. */
enum pkda_gate_kind {
  PKDA_GATE_LOG_HEAD = 0,    /* g [N_tok, H]    log-decay per token and head          */
  PKDA_GATE_LOG_CHANNEL = 1, /* g [N_tok, H, K] log-decay per key channel             */
  PKDA_GATE_RAW_CHANNEL = 2, /* g [N_tok, H, K] raw; -exp(A_log[h]) softplus(g + dt_bias[h,c]) */
  PKDA_GATE_LOW_RANK = 3     /* g = decay hidden [N_tok, rank] (row stride g_stride); the raw
                                gate is g up_weight^T [N_tok, H*K], rounded to g's dtype,
                                then activated as PKDA_GATE_RAW_CHANNEL */
};

/* ---------------------------------------------------------------------------
 * Library identity.
 * ------------------------------------------------------------------------- */
int pkda_abi_version(void);
const char* pkda_last_error(void);
/* sizeof() of each argument struct, so a binding can check its mirror. */
int64_t pkda_args_size(int which);
enum pkda_args_kind {
  PKDA_ARGS_RECURRENT = 0,
  PKDA_ARGS_GATE = 1,
  PKDA_ARGS_PRECOND = 2,
  PKDA_ARGS_CHUNK_FWD = 3,
  PKDA_ARGS_CHUNK_BWD = 4,
  PKDA_ARGS_QKV_CONV = 5,
  PKDA_ARGS_NORM_GATE = 6,
  PKDA_ARGS_CONTROLS = 7
};

/* ---------------------------------------------------------------------------
 * Token-recurrent forward and the slot-pool decode step.
 *
 * Replaces FLA's fused_recurrent_precond_kda as called by
 * PreconditionedKDA._cuda_recurrence (delta_feedback_experiment/pkda.py:473-474)
 * and adds the in-place slot-pool decode form.  One workgroup per
 * (sequence, head) holds that head's FP32 state in registers for all of the
 * sequence's tokens; the state is read once and written once.
 *
 * Sequences: cu_seqlens given -> num_seqs packed documents; otherwise
 * num_seqs rows of seqlen tokens each (decode: seqlen = 1).
 * State source, per sequence n (slot s = slot_idx ? slot_idx[n] : n):
 *   state_pool != NULL: S = state_pool[s] (pool [pool_size, H, K, V] FP32) and
 *                       the final state is written back to state_pool[s]
 *                       (in place; slots must be unique -- the host checks
 *                       range and uniqueness only when check_slots != 0);
 *   else S = initial_state ? initial_state[n] : 0, and the final state goes
 *        to final_state[n] when final_state != NULL.
 * The preconditioner state follows the same rule with a_pool /
 * initial_A_state / final_A_state ([.., H, K] FP32).
 * ------------------------------------------------------------------------- */
typedef struct pkda_recurrent_args {
  int32_t struct_size;   /* sizeof(pkda_recurrent_args) */
  int32_t dtype;         /* pkda_dtype of q, k, v, o */
  int32_t num_seqs, seqlen, heads, head_dim;
  const int32_t* cu_seqlens; /* [num_seqs+1] or NULL */
  const void* q;         /* [N_tok, H, K] */
  const void* k;         /* [N_tok, H, K] */
  const void* v;         /* [N_tok, H, V] */
  const void* g;         /* see gate_kind */
  int32_t gate_kind;     /* pkda_gate_kind */
  int32_t g_dtype;       /* pkda_dtype of g */
  const float* A_log;    /* [H]    (PKDA_GATE_RAW_CHANNEL) */
  const float* dt_bias;  /* [H*K]  (PKDA_GATE_RAW_CHANNEL) */
  const float* beta;     /* [N_tok, H] */
  float scale;
  /* preconditioner; disabled when g_atk == NULL */
  const float* g_atk;    /* [N_tok, H] log-decay */
  const float* beta_atk; /* [N_tok, H] */
  const float* center;   /* [H] (log_atk_scale) */
  float squash_x, squash_eps;
  /* state */
  float* state_pool;          /* [pool_size, H, K, V] or NULL */
  float* a_pool;              /* [pool_size, H, K] or NULL */
  int64_t pool_size;
  const int32_t* slot_idx;    /* [num_seqs] device, or NULL (identity) */
  const int32_t* slot_idx_host; /* optional host copy for check_slots */
  int32_t check_slots;
  const float* initial_state;   /* [num_seqs, H, K, V] or NULL */
  const float* initial_A_state; /* [num_seqs, H, K] or NULL */
  float* final_state;           /* [num_seqs, H, K, V] or NULL */
  float* final_A_state;         /* [num_seqs, H, K] or NULL */
  void* o;                      /* [N_tok, H, V] in dtype */
} pkda_recurrent_args;

int pkda_recurrent_fwd(const pkda_recurrent_args* args, void* stream);
/* Same kernel; requires seqlen == 1 and state_pool != NULL. */
int pkda_decode_step(const pkda_recurrent_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Chunk geometry for packed documents.
 *
 * Chunks of PKDA_CHUNK tokens start at every document's first token.  With
 * cu_seqlens the chunk list depends on the data, so it is built on the device
 * into a caller-provided int32 workspace `table` of
 *   4 * num_chunks_max + 3 * num_seqs + 3 elements
 * (per chunk {document, first token, length, -}; each document's first chunk
 * id plus the total; the documents ordered by length, longest first: the
 * per-document passes start the longest documents first; a sanitised copy of
 * cu_seqlens; a flag), num_chunks_max >= ceil(num_tokens / 64) + num_seqs (an
 * upper bound the host knows without reading cu_seqlens).  Every chunked
 * entry point below takes the same table and reads document bounds only from
 * its sanitised copy: the running maximum of cu_seqlens clamped to
 * [0, num_tokens].  A malformed cu_seqlens (cu[0] != 0, a decrease, or
 * cu[num_seqs] != num_tokens) therefore cannot move an access outside the
 * token tensors or the table; it sets the flag (the table's last element) to
 * 1, which a caller may read back.  Launches sized by num_chunks_max skip the
 * unused tail.  Equal-length rows need no table (pass NULL).
 * pkda_recurrent_fwd reads cu_seqlens directly: pass it the table's
 * sanitised copy (at 4 * num_chunks_max + 2 * num_seqs + 1) when the values
 * are not known to be well formed.
 * ------------------------------------------------------------------------- */
int pkda_chunk_table(const int32_t* cu_seqlens, int32_t num_seqs, int32_t num_tokens, int32_t num_chunks_max,
                     int32_t* table, void* stream);

/* ---------------------------------------------------------------------------
 * Gate: chunk-local cumulative log-decay, and its backward.
 *
 * Replaces FLA's kda_gate_chunk_cumsum / kda_gate_bwd as driven by
 * delta_feedback_experiment/fla_ops.py:290-299,423-432,480-487 (FLA works in
 * log2; this library keeps natural log throughout).
 *   forward:  gcum[t] = sum_{s in chunk, s <= t} glog[s], glog per gate_kind;
 *             gcum is [N_tok, H] (PKDA_GATE_LOG_HEAD) or [N_tok, H, K] FP32.
 *   backward: from dgcum (same shape as gcum) writes dg (same shape as g,
 *             FP32), and for PKDA_GATE_RAW_CHANNEL dA_log [H] and
 *             ddt_bias [H*K] through per-chunk partials dA_log_part
 *             [num_chunks, H] and ddt_bias_part [num_chunks, H*K]
 *             (caller workspace; summed in a fixed order -> deterministic).
 * ------------------------------------------------------------------------- */
typedef struct pkda_gate_args {
  int32_t struct_size;
  int32_t num_seqs, seqlen, heads, head_dim, gate_kind, g_dtype;
  const int32_t* cu_seqlens;
  const void* g;
  const float* A_log;
  const float* dt_bias;
  float* gcum;              /* forward output */
  const float* dgcum;       /* backward input */
  void* dg;                 /* backward output in dg_dtype, shape of g; PKDA_GATE_LOW_RANK: the
                               gradient of the raw gate [N_tok, H, K] (the host turns it into
                               the decay hidden's and up_weight's gradients with two GEMMs) */
  float* dA_log_part;       /* [num_chunks, H]   workspace (raw and low-rank gates) */
  float* ddt_bias_part;     /* [num_chunks, H*K] workspace (raw and low-rank gates) */
  float* dA_log;            /* [H]   (raw and low-rank gates) */
  float* ddt_bias;          /* [H*K] (raw and low-rank gates) */
  int32_t num_chunks;       /* chunks (equal rows) or num_chunks_max (packed) */
  const int32_t* table;     /* pkda_chunk_table output or NULL */
  /* PKDA_GATE_LOW_RANK: the decay expansion (decay_up, delta_feedback_experiment/
   * pkda.py:168,334-339) fused into the gate: up_weight [H*K, rank] in g_dtype,
   * rank 64 or 128 (== head_dim as in the reference), g_stride >= rank. */
  const void* up_weight;
  int32_t rank;
  int32_t g_stride;
  int32_t dg_dtype;         /* PKDA_F32 (0), or g_dtype for the per-channel forms */
  /* Forward, optional (per-channel forms: PKDA_GATE_LOG_CHANNEL, RAW_CHANNEL,
   * LOW_RANK): the cumsum is then formed in FP64 and split as gcum (its FP32
   * rounding) + gcum_lo (the FP32 rounding of the remainder), [N_tok, H, K].
   * Differences of cumsums (the decay between two tokens of a chunk) taken
   * as (gcum[t] - gcum[s]) + (gcum_lo[t] - gcum_lo[s]) then carry only their
   * own rounding, where gcum alone carries that of the larger cumsums
   * (~1e-5 of the difference once |gcum| reaches a few hundred).  NULL: FP32
   * cumsum, gcum only. */
  float* gcum_lo;
} pkda_gate_args;

int pkda_gate_fwd(const pkda_gate_args* args, void* stream);
int pkda_gate_bwd(const pkda_gate_args* args, void* stream);

/* pkda_gate_bwd without a caller workspace.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture that may not allocate, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as pkda_gate_bwd except that
 * dA_log_part / ddt_bias_part are ignored: the per-chunk partials go to a
 * static device array of PKDA_GATE_BWD_NOALLOC_MAX_FLOATS floats (16 MiB),
 * one per device, held until the process ends.  Calls with
 * num_chunks * heads * (head_dim + 1) above that return PKDA_ERANGE; the call
 * allocates nothing.  Every call on one device shares that device's array,
 * so calls that overlap on one device (concurrent streams, threads) race;
 * serialise them.  Each call writes every partial it reads, so nothing left
 * by an earlier call leaks into a result. */
#define PKDA_GATE_BWD_NOALLOC_MAX_FLOATS ((int64_t)1 << 22)
int pkda_gate_bwd_noalloc(const pkda_gate_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Preconditioner scan (forward) and its reverse scan (backward).
 *
 * Replaces FLA's ATK scans (chunk_atk_fwd / its backward) run inside
 * chunk_precond_kda_fwd/_bwd (delta_feedback_experiment/fla_ops.py:300-339,
 * 441-479); math of delta_feedback_experiment/pkda.py:392-398.
 *   forward:  kw [N_tok,H,K] (dtype), A at every chunk start a_chunk
 *             [num_chunks, H, K] FP32 (backward checkpoint), final A.
 *   backward: dkw ([N_tok,H,K], FP32 or dtype: grad_dtype) -> dk (accumulated:
 *             dk += ..., or written to dk_final),
 *             dg_atk, dbeta_atk [N_tok,H] FP32, dcenter [H] (through
 *             per-document partials dcenter_part [num_seqs, H], summed in a
 *             fixed order), dA0 [N,H,K] when dA0 != NULL; dA_T optional
 *             gradient of the final A.
 * Both scans run chunk-parallel: per (chunk, head) the chunk's local end
 * value, per (document, head) a scan over the document's chunks, per
 * (chunk, head) the chunk again from the value entering it.  a_chunk is that
 * scan's buffer in the forward (A entering each chunk on return) and
 * lam_chunk in the backward; the backward recomputes A inside each chunk
 * from a_chunk.  Packed documents take the pkda_chunk_table `table` (NULL
 * for equal rows).
 * ------------------------------------------------------------------------- */
typedef struct pkda_precond_args {
  int32_t struct_size;
  int32_t dtype;            /* of k and kw */
  int32_t num_seqs, seqlen, heads, head_dim;
  const int32_t* cu_seqlens;
  const void* k;
  const float* g_atk;
  const float* beta_atk;
  const float* center;
  float squash_x, squash_eps;
  const float* initial_A_state;  /* [N,H,K] or NULL */
  float* final_A_state;          /* [N,H,K] or NULL */
  void* kw;                      /* forward output [N_tok,H,K] dtype */
  float* a_chunk;                /* [num_chunks, H, K] */
  int32_t num_chunks;
  const void* dkw;               /* backward input, grad_dtype */
  void* dk;                      /* backward: accumulated into (FP32), or read only (grad_dtype
                                    narrower than FP32, with dk_final) */
  float* dg_atk;
  float* dbeta_atk;
  float* dcenter_part;           /* [num_chunks, H] workspace */
  float* dcenter;                /* [H] */
  float* dA0;                    /* [N,H,K] or NULL */
  const float* dA_T;             /* [N,H,K] or NULL */
  const int32_t* table;          /* pkda_chunk_table output or NULL */
  /* forward only: slot-indexed A states, as pkda_chunk_fwd_args.slot_idx
   * (initial_A_state / final_A_state are then [pool_size, H, K]) */
  const int32_t* slot_idx;
  int64_t pool_size;
  float* lam_chunk;              /* backward workspace [num_chunks, H, K] */
  void* dk_final;                /* backward, optional: dk + the preconditioner's terms
                                    written here in dtype, dk left as it came in */
  float* kw32;                   /* forward, optional: kw [N_tok,H,K] also in FP32 (the
                                    chunk backward's exact in-block pair sums read it) */
  int32_t grad_dtype;            /* backward: dtype of dkw and dk, PKDA_F32 or `dtype`; the
                                    narrow form needs dk_final (the chunk backward hands its
                                    key gradients over in the activation dtype: half the bytes
                                    for it to write and for both reverse-scan passes to read) */
  float* chunk_decay;            /* optional workspace [num_chunks, H] FP32: each chunk's
                                    exp(sum of g_atk), written by the local chunk pass and read
                                    by the document scan (which otherwise sums every chunk's
                                    g_atk again); the same bits either way */
} pkda_precond_args;

int pkda_precond_fwd(const pkda_precond_args* args, void* stream);
int pkda_precond_bwd(const pkda_precond_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Kernel stages of the chunked entry points.  `stages` selects which of an
 * entry point's kernels one call enqueues (0 = all, in order).  A caller that
 * splits a call into stages must issue them in the listed order on one stream;
 * the split exists so that each kernel can be timed or placed on its own.
 * ------------------------------------------------------------------------- */
enum pkda_chunk_stage {
  PKDA_STAGE_ALL = 0,
  PKDA_STAGE_FWD_INTRA = 1, /* per chunk: Akk, T = (I + Akk)^-1, Aqk (w, u)   */
  PKDA_STAGE_FWD_STATE = 2, /* per document: U, o, the chunk states h, S_T     */
  PKDA_STAGE_BWD_STATE = 1, /* per document, reverse: dh, dU, dS0            */
  PKDA_STAGE_BWD_CHUNK = 2  /* per chunk: every gradient of the chunk          */
};

/* ---------------------------------------------------------------------------
 * Chunked forward (training / prefill).
 *
 * Replaces chunk_precond_kda_fwd as called by the pkda_recurrence custom op
 * (delta_feedback_experiment/fla_ops.py:316-339) and by chunk_precond_kda
 * (delta_feedback_experiment/pkda.py:475).  Inputs are the gate's gcum and the
 * preconditioner's kw (kw == k when there is no preconditioner).
 * Per chunk: Akk (strictly lower, row = read key, col = write key),
 * T = (I + Akk)^-1, w = T diag(beta) (exp(gcum) * k), u = T diag(beta) v,
 * Aqk (inclusive, with `scale`); per document, sequentially over chunks:
 * U = u - w S, o = (exp(gcum) * scale q) S + Aqk U, S <- exp(gcum_last) S + kg^T U.
 * Saved for the backward (all [N_tok, H, *] in dtype unless stated):
 * w, u (overwritten with U), aqk [.., 64], akk (= T) [.., 64],
 * h [num_chunks, H, K, V] (state entering each chunk; NULL when not training).
 * BF16 with a per-head gate never stores w (it may be NULL, here and in the
 * backward) nor the intermediate u: its state passes form U = T diag(beta)
 * (v - exp(gcum) * (k S)) and w^T dU = k^T diag(beta exp(gcum)) T^T dU from
 * akk, k and v, and u receives U alone.
 * Per-channel gates (gate_per_channel != 0, gcum [N_tok, H, K]): the decay
 * sits inside every key contraction.  Pairs of tokens in different 16-token
 * sub-blocks are products of operands each scaled by a decay <= 1 relative
 * to the last token before the row's sub-block (no overflow for any gate);
 * pairs inside one sub-block are summed exactly, channel by channel.  The
 * gated operands qg = scale e^G q and kg = e^{G_last - G} kw [N_tok, H, K]
 * (dtype) are written for the state pass and the backward.
 * ------------------------------------------------------------------------- */
typedef struct pkda_chunk_fwd_args {
  int32_t struct_size;
  int32_t dtype;
  int32_t num_seqs, seqlen, heads, head_dim;
  const int32_t* cu_seqlens;
  int32_t num_chunks;
  const int32_t* table;
  const void *q, *k, *kw, *v;
  const float* gcum;
  int32_t gate_per_channel;
  const float* beta;
  float scale;
  const float* initial_state;  /* [N,H,K,V] or NULL */
  float* final_state;          /* [N,H,K,V] or NULL */
  void* o;
  void *w, *u, *aqk, *akk, *h;
  int32_t stages;              /* pkda_chunk_stage mask, 0 = all */
  void *qg, *kg;               /* per-channel gates only, else NULL */
  /* Slot-indexed states (cached prefill into a decode pool): when slot_idx
   * (int32 [num_seqs], device) is given, document n starts from
   * initial_state[slot_idx[n]] (zero when initial_state is NULL) and leaves its
   * final state in final_state[slot_idx[n]]; both are then
   * [pool_size, H, K, V] and may be the same pool (in place: slots must be
   * unique).  NULL: document n uses row n. */
  const int32_t* slot_idx;
  int64_t pool_size;
  /* Optional, FP32 with a per-channel gate: the gate's gcum_lo
   * (pkda_gate_args.gcum_lo).  The pair decays e^{G[t]-G[s]} inside a chunk
   * are then formed from (gcum[t] - gcum[s]) + (gcum_lo[t] - gcum_lo[s]).
   * Ignored for BF16.  NULL: gcum alone. */
  const float* gcum_lo;
  /* Nonzero (BF16, per-head gate, kw == k or NULL only): aqk and akk hold
   * each chunk's ten 16 x 16 blocks on and below the diagonal, packed
   * [num_chunks, H, 10, 16, 16] (blocks in the order (0,0) (1,0) (1,1) (2,0)
   * (2,1) (2,2) (3,0) .. (3,3), each row-major; rows past a chunk's end zero)
   * instead of [N_tok, H, 64]: 5 KB instead of 8 KB per chunk and head to
   * write and to read back.  The backward takes the same flag. */
  int32_t tri_packed;
} pkda_chunk_fwd_args;

int pkda_chunk_fwd(const pkda_chunk_fwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Chunked backward.
 *
 * Replaces chunk_precond_kda_bwd (delta_feedback_experiment/fla_ops.py:441-479)
 * for the recurrence proper (the gate and preconditioner backward are the
 * entry points above).  Consumes the forward's saved tensors and do
 * (and dht, the final-state gradient, or NULL).  Workspace (caller):
 * dh [num_chunks, H, K, V] and du [N_tok, H, V], both in dtype.  Outputs:
 * dq, dv in grad_dtype and dk (read key), dkw (write key; when kw == k it is
 * added into dk and may be NULL) in key_grad_dtype (FP32, or dtype when the
 * caller wants the input dtype directly; FP32 key gradients with dtype dq, dv
 * for a caller that accumulates the preconditioner's terms into dk and dkw);
 * dbeta [N_tok,H], dgcum (shape of gcum), dh0 [N,H,K,V] (NULL if not wanted)
 * in FP32.
 * ------------------------------------------------------------------------- */
typedef struct pkda_chunk_bwd_args {
  int32_t struct_size;
  int32_t dtype;
  int32_t num_seqs, seqlen, heads, head_dim;
  const int32_t* cu_seqlens;
  int32_t num_chunks;
  const int32_t* table;
  const void *q, *k, *kw, *v;
  const float* gcum;
  int32_t gate_per_channel;
  const float* beta;
  float scale;
  const float* initial_state;
  const void *w, *u, *aqk, *akk, *h;
  const void* do_;
  const float* dht;
  void* dh;
  void* du;
  void *dq, *dk, *dkw, *dv;     /* dq, dv in grad_dtype; dk, dkw in key_grad_dtype */
  float *dbeta, *dgcum, *dh0;
  int32_t stages;              /* pkda_chunk_stage mask, 0 = all */
  const void *qg, *kg;         /* per-channel gates only: the forward's qg, kg */
  int32_t grad_dtype;          /* dq, dv: PKDA_F32 or dtype (one rounding of the FP32 value) */
  int32_t key_grad_dtype;      /* dk, dkw: grad_dtype, or PKDA_F32 when grad_dtype is dtype */
  /* Optional, per-channel gates with a separate write key in BF16: kw in FP32
   * [N_tok,H,K] (pkda_precond_args.kw32).  The gate gradient's largest terms
   * are the in-block query/key pairs, summed exactly; formed from the BF16
   * write key they move dA_log (a sum of the gate gradient over a whole head)
   * by ~1e-2.  NULL: the BF16 kw serves. */
  const float* kw32;
  /* Optional, FP32 with a per-channel gate: as pkda_chunk_fwd_args.gcum_lo.
   * The gate gradient sums the pair terms of a chunk with the decays between
   * the pair's tokens inside them; with gcum alone their FP32 rounding moves
   * dA_log (a signed sum of that gradient over a whole head) by ~1e-5. */
  const float* gcum_lo;
  int32_t tri_packed;          /* as pkda_chunk_fwd_args.tri_packed: how the forward stored aqk, akk */
} pkda_chunk_bwd_args;

int pkda_chunk_bwd(const pkda_chunk_bwd_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * Fused Q/K/V short convolution + SiLU + per-head L2 normalisation.
 *
 * Replaces delta_feedback::pkda_qkv_conv and its backward op
 * (delta_feedback_experiment/fla_ops.py:134-249), the producer of the
 * recurrence's q, k, v (portable form: delta_feedback_experiment/pkda.py:
 * 37-44,197-220,290-316).  x [batch, seqlen, 3 * width] holds the Q, K and V
 * projections side by side; weight [3 * width, conv_size] is the depthwise
 * causal filter (zero history before the first token).  Per channel c:
 *   y = silu(sum_w weight[c, w] x[t - (conv_size - 1) + w, c]),
 * then for c < norm_channels (Q and K) y / sqrt(sum over the head_dim channels
 * of c's head of y^2 + eps); FP32 throughout, cast once to dtype.
 *   forward:  q, k, v [batch, seqlen, width] (dtype).
 *   backward: from dq, dk, dv (dtype): dx (dtype, shape of x) and dw (w_dtype,
 *             shape of weight) through the caller's FP32 workspace dw_part of
 *             pkda_qkv_conv_workspace(batch, seqlen, width, conv_size)
 *             elements, summed in a fixed order (deterministic).
 * head_dim 32, 64 or 128; conv_size 1..4; width a multiple of head_dim.
 *
 * Cached rows (forward only; the decode-time counterpart of the reference's
 * conv_state, delta_feedback_experiment/pkda.py:240-260): history_in
 * [pool_size, conv_size - 1, 3 * width] (dtype) holds, per slot, the raw
 * projections of the conv_size - 1 positions before the row's first token
 * (oldest first; zero history when NULL); history_out (same shape, may be
 * history_in itself) receives the last conv_size - 1 rows of history ++ x.
 * Row b uses slot slot_idx[b] (int32 [batch], device; row b when NULL).
 * ------------------------------------------------------------------------- */
typedef struct pkda_qkv_conv_args {
  int32_t struct_size;
  int32_t dtype;            /* of x, q, k, v, dq, dk, dv, dx */
  int32_t w_dtype;          /* of weight and dw */
  int32_t batch, seqlen, width, head_dim, norm_channels, conv_size;
  float eps;
  const void* x;
  const void* weight;
  void *q, *k, *v;          /* forward outputs */
  const void *dq, *dk, *dv; /* backward inputs */
  void* dx;                 /* backward outputs */
  void* dw;
  float* dw_part;           /* backward workspace */
  const int32_t* slot_idx;  /* cached rows, forward only (see above) */
  const void* history_in;
  void* history_out;
  int64_t pool_size;
} pkda_qkv_conv_args;

int64_t pkda_qkv_conv_workspace(int32_t batch, int32_t seqlen, int32_t width, int32_t conv_size);
int pkda_qkv_conv_fwd(const pkda_qkv_conv_args* args, void* stream);
int pkda_qkv_conv_bwd(const pkda_qkv_conv_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * RMSNorm with a sigmoid output gate, the consumer of the recurrence output.
 *
 * Replaces delta_feedback::pkda_norm_gate and its backward op
 * (delta_feedback_experiment/fla_ops.py:572-657), as
 * PreconditionedKDA.forward applies it to o [B, T, H, d] with the gate logits
 * and output_norm (delta_feedback_experiment/pkda.py:536-547).  Per row r of
 * width dim (one head of one token), in FP32 with one rounding:
 *   rstd[r] = 1 / sqrt(mean(x[r]^2) + eps),
 *   y[r]    = x[r] rstd[r] weight sigmoid(gate[r]).
 *   forward:  y (dtype), rstd [rows] FP32.
 *   backward: from dy (dtype) and the forward's rstd: dx, dgate (dtype) and
 *             dweight (w_dtype) through the caller's FP32 workspace dw_part
 *             of pkda_norm_gate_workspace(rows, dim) elements, summed in a
 *             fixed order (deterministic).
 * x, gate, y, dy, dx, dgate share dtype; dim 64 or 128.
 * ------------------------------------------------------------------------- */
typedef struct pkda_norm_gate_args {
  int32_t struct_size;
  int32_t dtype;       /* of x, gate, y, dy, dx, dgate */
  int32_t w_dtype;     /* of weight and dweight */
  int32_t dim;
  int64_t rows;
  float eps;
  const void* x;
  const void* gate;
  const void* weight;  /* [dim] */
  void* y;             /* forward outputs */
  float* rstd;         /* forward output, backward input: [rows] */
  const void* dy;      /* backward input */
  void* dx;            /* backward outputs */
  void* dgate;
  void* dw;
  float* dw_part;      /* backward workspace */
} pkda_norm_gate_args;

int64_t pkda_norm_gate_workspace(int64_t rows, int32_t dim);
int pkda_norm_gate_fwd(const pkda_norm_gate_args* args, void* stream);
int pkda_norm_gate_bwd(const pkda_norm_gate_args* args, void* stream);

/* ---------------------------------------------------------------------------
 * PKDA control activations and their packed gradient.
 *
 * Replaces the activation half of PreconditionedKDA._controls
 * (delta_feedback_experiment/pkda.py:318-353) and, backward, the
 * _PackedControlSplit backward with pack_control_gradients
 * (delta_feedback_experiment/pkda.py:56-74, cuda_kernels.py:1081-1172).
 * packed [rows, row_stride] (dtype) holds per token the five control
 * projections side by side (width = rank + 3 H + gate_width columns):
 *   decay hidden [rank] | beta logits [H] | preconditioner decay logits [H] |
 *   preconditioner beta logits [H] | output-gate hidden [gate_width].
 *   forward:  beta = sigmoid(beta logit), precond_beta = sigmoid(its logit)
 *             (dtype, [rows, H]); precond_decay = -exp(A_log_p[h])
 *             softplus(logit + dt_bias_p[h]) (FP32, [rows, H]).  The two
 *             hidden slices stay where they are (the caller's views).
 *   backward: from d_decay_hidden [rows, rank], dbeta, dprecond_beta
 *             [rows, H] (dtype), dprecond_decay [rows, H] (FP32) and
 *             d_gate_hidden [rows, gate_width] (dtype; any may be NULL for a
 *             zero gradient), dpacked [rows, width] (dtype, contiguous) in one
 *             pass, with the sigmoid and softplus derivatives applied; and
 *             dA_log_p [H], ddt_bias_p [H] (FP32) through the caller's FP32
 *             workspace part of pkda_controls_workspace(rows, H) elements,
 *             summed in a fixed order (deterministic).
 * The sigmoid outputs are taken as rounded to dtype, as the reference's
 * tensors are, in both directions.
 * ------------------------------------------------------------------------- */
typedef struct pkda_controls_args {
  int32_t struct_size;
  int32_t dtype;              /* of packed, beta, precond_beta and the dtype gradients */
  int64_t rows;
  int32_t heads, rank, gate_width, row_stride;
  const void* packed;
  const float* A_log_p;       /* [H] */
  const float* dt_bias_p;     /* [H] */
  void* beta;                 /* forward outputs */
  float* precond_decay;
  void* precond_beta;
  const void* d_decay_hidden; /* backward inputs */
  const void* dbeta;
  const float* dprecond_decay;
  const void* dprecond_beta;
  const void* d_gate_hidden;
  void* dpacked;              /* backward outputs */
  float* part;
  float* dA_log_p;
  float* ddt_bias_p;
} pkda_controls_args;

int64_t pkda_controls_workspace(int64_t rows, int32_t heads);
int pkda_controls_fwd(const pkda_controls_args* args, void* stream);
int pkda_controls_bwd(const pkda_controls_args* args, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PKDA_GFX950_H */
