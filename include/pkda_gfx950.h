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
 *    host and keeps no state besides the last error message, so a caller may
 *    capture every call into a HIP graph.
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

#define PKDA_ABI_VERSION 1
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
  PKDA_GATE_RAW_CHANNEL = 2  /* g [N_tok, H, K] raw; -exp(A_log[h]) softplus(g + dt_bias[h,c]) */
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
  PKDA_ARGS_CHUNK_BWD = 4
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

#ifdef __cplusplus
}
#endif
#endif /* PKDA_GFX950_H */
