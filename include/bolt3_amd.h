/*
 * bolt3_amd — C ABI of the MI355X (gfx950) Bolt-3 Dual-Field attention kernels.
 *
 * Each entry point replaces a group of PyTorch ops of the reference's pure
 * Python implementation (vsa_lm/config/bolt3.py, cited per function below).
 * Conventions shared by all entry points:
 *   - arguments come in one plain struct of device pointers, element strides and
 *     sizes; no allocation, no host synchronisation, no exceptions;
 *   - `stream` is a hipStream_t passed as void*; work is enqueued on it only;
 *   - return 0 on success, a positive B3_ERR_* domain code for a rejected
 *     argument, or a hipError_t code from the launch;
 *   - storage dtype is B3_F32 or B3_BF16 (raw bf16 bits); slot masses, utilities,
 *     positions, gates and M_res are always fp32.
 * Layout names: B batch rows, H query heads, HKV key/value heads, HD head dim,
 * S attractor slots, C chunk length, bh = b*HKV + hkv.
 */
#ifndef BOLT3_AMD_H
#define BOLT3_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { B3_F32 = 0, B3_BF16 = 1 };
enum { B3_OK = 0, B3_ERR_ARG = 1001, B3_ERR_UNSUPPORTED = 1002, B3_ERR_WORKSPACE = 1003 };

/* Rows of one decision-log record (per step, per bh, B3_LOG_COLS floats each). */
enum {
  B3_LOG_REL = 0,      /* rel_err per token                          */
  B3_LOG_SCORE = 1,    /* eviction / fill score per token            */
  B3_LOG_BEST = 2,     /* best slot cosine per token (steady)        */
  B3_LOG_SIMV = 3,     /* value cosine with the best slot (steady)   */
  B3_LOG_SLOT = 4,     /* argmax slot per token (steady)             */
  B3_LOG_MERGE = 5,    /* 1 if merged                                */
  B3_LOG_DELTA = 6,    /* 1 if written to M_res                      */
  B3_LOG_TOPTOK = 7,   /* token order (steady: candidates; fill: picked) */
  B3_LOG_BOTSLOT = 8,  /* slot order by keep, ascending (steady)     */
  B3_LOG_WIN = 9,      /* 1 if the i-th pair (token, slot) swapped   */
  B3_LOG_KEEP = 10,    /* keep value per slot                        */
  B3_LOG_TOPVAL = 11,
  B3_LOG_BOTVAL = 12,
  B3_LOG_INFO = 13,    /* column 0: B3_TIE_* bits of the step         */
  B3_LOG_ROWS = 14,
  B3_LOG_COLS = 256
};

/* Tie handling of a consolidation step (B3_LOG_INFO, column 0).  Orderings are ranks; where
 * exactly equal values decide which token takes which slot, the order among them is the
 * reference's torch.topk order on the CPU (nth_element + sort, or partial_sort), restated. */
enum {
  B3_TIE_TOP = 1,      /* equal candidate (or fill) scores in the deciding prefix: reference order used */
  B3_TIE_BOT = 2,      /* equal keep values in the deciding prefix: reference order used */
  B3_TIE_LIMIT = 4     /* the library's depth-limit heap fallback would run: order not restated */
};

/* [B][heads][t][HD] output view: element (b, h, t, d) at p + b*sb + h*sh + t*HD + d. */
typedef struct { void* p; int64_t sb, sh; } b3_tensor_out;
/* fp32 [B][heads][t] view: element (b, h, t) at p + b*sb + h*sh + t. */
typedef struct { float* p; int64_t sb, sh; } b3_gate_out;

typedef struct {
  int32_t dtype, B, T, H, HKV, HD;
  const void* lin;            /* [B][T][lin_row_stride]: q | k | v | beta | eta columns (projection output),
                                 or q | eta columns when lin_kv is set; rows and head outputs 16-byte aligned */
  int64_t lin_row_stride;
  const void* lin_kv;         /* optional [B][T][lin_kv_row_stride]: k | v | beta columns (a separate projection) */
  int64_t lin_kv_row_stride;
  int32_t parts;              /* 1: q heads and eta only; 2: k/v heads, beta and pos_out only; 0 or 3: all */
  const float* qn_w;          /* [HD] q RMSNorm weight (fp32 values) or NULL */
  const float* kn_w;          /* [HD] k RMSNorm weight or NULL */
  int32_t has_qk_norm;
  float eps;
  const float* inv_freq;      /* [HD/2] RoPE inverse frequencies (fp32 values of the module buffer) */
  int32_t pos0;               /* position of row t is pos0 + t */
  b3_tensor_out q_raw, q_rope, k_raw, k_rope, v;  /* q_raw / k_raw may have p == NULL */
  b3_gate_out beta, eta;      /* sigmoid / tanh gates, values rounded to the storage dtype */
  float* pos_out;             /* optional fp32 [T]: pos0 + t */
  const void* gates;          /* optional [B][T][gates_row_stride]: beta (HKV) | eta (H) projection columns;
                                 when set, the gates are read here instead of from lin / lin_kv */
  int64_t gates_row_stride;
  uint32_t* rope_cs;          /* optional, bf16 only: [T][HD/2] the rounded (cos, sin) of position pos0 + t and
                                 frequency i, cos in the low 16 bits -- the table b3_attn_args.rope_cs reads */
} b3_heads_args;

/*
 * Head preparation for a block of tokens: q/k RMSNorm, RoPE, beta/eta gates.
 * Replaces head_qkv's norms + LlamaRoPE + gates:
 * vsa_lm/config/bolt3.py:59-66 (head_qkv), :197-199 (forward) and :346-349 (step);
 * vsa_lm/surgery.py:49-53 (LlamaRMSNorm), :86-93 (LlamaRoPE).
 */
int bolt3_heads(const b3_heads_args* a, void* stream);

typedef struct {
  int32_t dtype, B, HKV, HD, S;
  /* consolidated tokens: element (bh, n, d) at kr + bh*tok_bh_stride + n*HD + d (same for kp, v) */
  const void* kr;             /* un-roped keys   */
  const void* kp;             /* roped keys      */
  const void* v;
  int64_t tok_bh_stride;
  const float* pos;           /* fp32 position of token n (shared by all bh) */
  const float* beta;          /* fp32 (bh, n) at beta + bh*beta_bh_stride + n */
  int64_t beta_bh_stride;
  int32_t n_steps;            /* consolidations run back to back                          */
  int32_t off0, len0;         /* step 0 consumes tokens [off0, off0 + len0)               */
  int32_t step_stride, step_len; /* step i > 0 consumes [i*step_stride, i*step_stride + step_len) */
  int32_t n_filled;           /* filled slots before step 0; 0: the chain starts from the empty state
                                 (zero slots, mass 1, M_res 0) and the state arrays are outputs only */
  int32_t kp_exact;           /* 1: kp rows are bolt3_heads / bolt3_decode RoPE of kr at pos (bit-exact),
                                 so a slot taken from a token copies its roped key; 0: recompute */
  /* slot state, updated in place: ak/av [bh][S][HD] storage dtype (un-roped keys), mass/util/pm [bh][S],
     act [bh][S] (0/1), m_res [bh][HD][HD] */
  void* ak;
  void* av;
  float* mass;
  float* util;
  float* pm;
  uint8_t* act;
  float* m_res;
  const float* kappa;         /* [HKV] */
  const float* gamma;         /* [HKV] M_res decay */
  const float* inv_freq;      /* [HD/2] */
  /* optional outputs after every step (NULL to skip), packed per step: snap_k / snap_v
     [n_steps][B*HKV][S][HD] roped slot keys and slot values (storage dtype), snap_bias
     [n_steps][B*HKV][S] attention bias kappa*log(max(mass,1)) (-inf for inactive slots),
     snap_m [n_steps][B*HKV] blocks of HD*HD floats holding M_res: fp32 storage M[c][d];
     bf16 storage M^T[d][c] split into bf16 hi followed by bf16 lo */
  void* snap_k;
  void* snap_v;
  float* snap_bias;
  float* snap_m;
  float* log;                 /* optional decision log [n_steps][bh][B3_LOG_ROWS][B3_LOG_COLS] */
  void* work;                 /* scratch of >= bolt3_chain_workspace_bytes(...) bytes */
  int64_t work_bytes;
  /* 0: the whole chain; 1: the slot decisions only (the slot state, snap_k / snap_v / snap_bias, the
     log and the delta-rule weights in `work`); 2: the Gershgorin scales and the M_res updates
     (m_res, snap_m) of the steps that a phase-1 call with the same arguments and the same `work`
     decided.  Phase 2 may run concurrently with the phase-1 call of the next steps when that call
     uses another `work` buffer. */
  int32_t phase;
  /* optional (NULL to skip): each slot-decision workgroup adds 1 to *started when it begins, so
     that bolt3_wait_count can hold another stream until all B*HKV of them hold a compute unit */
  uint32_t* started;
  /* optional (NULL to skip): the slots' mass and mean position after every step,
     [n_steps][B*HKV][S] fp32 each (the backward's record of merges and evictions) */
  float* snap_mass;
  float* snap_pm;
} b3_chain_args;

/*
 * Consolidation chain: n_steps successive _consolidate_functional calls per bh.
 * Three kernels on the stream: the slot decisions (one workgroup per bh, slot
 * state resident in LDS), the Gershgorin scales (one workgroup per step and bh)
 * and the M_res delta rule (one workgroup per bh and 32 columns of M).
 * Replaces vsa_lm/config/bolt3.py:68-192 (fill, score, merge, evict, Gershgorin
 * delta-rule M_res update) as driven by the chunk loop at :262-273 and by
 * Bolt3Decoder.step at :406-425.  Token lengths per step must be <= 256,
 * S == 128, HD in {64, 128}.
 */
int bolt3_chain(const b3_chain_args* a, void* stream);
/*
 * bolt3_chain without a caller workspace: the same kernels and results, with the workspace taken
 * from a scratch array of B3_CHAIN_NOALLOC_SCRATCH_BYTES that the library keeps on each GPU (held
 * until the process ends).  No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops).  a->work and
 * a->work_bytes are ignored; a launch whose bolt3_chain_workspace_bytes(...) exceeds the
 * scratch size is rejected with B3_ERR_WORKSPACE before anything runs.  Call it with the
 * stream's device current.  Every call on one GPU shares that GPU's scratch, so calls that
 * overlap on one GPU race (also a phase-2 call beside another phase-1 call); the scratch needs
 * no clearing (every byte the kernels read was written by the same call).  Allocates nothing.
 */
#define B3_CHAIN_NOALLOC_SCRATCH_BYTES (4 << 20)
int bolt3_chain_noalloc(const b3_chain_args* a, void* stream);

/* Workspace bytes for a launch of n_steps steps: per-step delta-rule weights and Gershgorin
   scales (3 x n_steps x B*HKV x 256 floats) plus, for fp32 storage with HD == 128, the roped
   slot keys (B*HKV x S x HD floats). */
int64_t bolt3_chain_workspace_bytes(int32_t dtype, int32_t B, int32_t HKV, int32_t HD, int32_t S, int32_t n_steps);

typedef struct {
  int32_t dtype, B, HKV, HD, S;
  const void* ak;             /* [bh][S][HD] un-roped slot keys (storage dtype) */
  const float* pm;            /* [bh][S] mean positions */
  const float* mass;          /* [bh][S] */
  const uint8_t* act;         /* [bh][S] */
  const float* kappa;         /* [HKV] */
  const float* inv_freq;      /* [HD/2] */
  void* slot_k;               /* out: [bh][S][HD] slot keys roped at their mean positions */
  float* slot_bias;           /* out: [bh][S] kappa*log(max(mass,1)), -inf where inactive */
} b3_slot_keys_args;

/*
 * The slot field's keys and bias as the attention reads them, from a slot state (with the
 * chain's own RoPE rounding).  The decoder keeps them cached and the chain refreshes them; this
 * rebuilds them for a state restored from the reference's kv_caches dict.
 * Replaces the attractor RoPE and bias of vsa_lm/config/bolt3.py:383-388 (recomputed there at
 * every step) and :236-241.  S == 128, HD in {64, 128}.
 */
int bolt3_slot_keys(const b3_slot_keys_args* a, void* stream);

/*
 * Holds `stream` until *counter has reached `target` (compared modulo 2^32) or after max_polls
 * polls (each a device-scope read and a short sleep), whichever comes first.  No counterpart in the reference (its chain
 * is serial host code): the forward launches the slot decisions (one workgroup per bh, each with
 * the whole LDS of a compute unit) on a side stream and calls this on its main stream, with
 * `counter` = b3_chain_args.started, before a full-chip GEMM, so that the GEMM's workgroups cannot
 * take every compute unit first and leave the slot decisions waiting for the GEMM's end.  One
 * 64-thread workgroup; counter is device memory.
 */
int bolt3_wait_count(const uint32_t* counter, uint32_t target, int32_t max_polls, void* stream);

typedef struct {
  int32_t dtype, B, H, HKV, HD, S, C, n_sinks;
  int32_t mode;               /* 0: every chunk of a forward; 1: one block of queries against decoder state */
  int32_t n_q;                /* queries per batch row (mode 0: T, mode 1: tokens in this step) */
  int32_t score_round;        /* 1: q.k rounded to the storage dtype before scaling (forward); 0: fp32 (step) */
  const void* q_rope;         /* (b, h, t, d) at + b*q_sb + h*q_sh + t*HD + d */
  const void* q_raw;
  int64_t q_sb, q_sh;
  const float* eta;           /* (b, h, t) at + b*e_sb + h*e_sh + t */
  int64_t e_sb, e_sh;
  const void* win_k;          /* (b, hkv, n, d) at + b*w_sb + hkv*w_sh + n*HD + d; roped keys */
  const void* win_v;
  int64_t w_sb, w_sh;
  int32_t a_start, a_len;     /* mode 1: older window segment [a_start, a_start + a_len) */
  int32_t b_start, b_len;     /* mode 1: current segment; query t is at segment index b_len - n_q + t */
  const void* sink_k;         /* mode 1: (b, hkv, n, d) at + b*s_sb + hkv*s_sh + n*HD + d */
  const void* sink_v;
  int64_t s_sb, s_sh;
  int32_t n_sink_keys;        /* mode 1: number of sink keys present (0 = none) */
  const void* slot_k;         /* [step][bh][S][HD] roped slot keys (mode 0: step = chunk - 2) */
  const void* slot_v;
  const float* slot_bias;     /* [step][bh][S] */
  int64_t slot_step;          /* elements between steps of slot_k / slot_v (bias: slot_step / HD) */
  int32_t has_slots;          /* mode 1 */
  const float* m_res;         /* [step][bh] blocks of HD*HD floats (mode 1: NULL = no readout) */
  int64_t m_step;             /* floats between steps */
  int32_t m_split;            /* 0: block is M[c][d] fp32; 1 (bf16 only): block is M^T[d][c] as bf16 hi
                                 then bf16 lo (the chain's snap_m layout for bf16 storage) */
  const float* gamma;         /* [HKV] */
  const float* res_w;         /* [HD] fp32 res_norm weight */
  float eps;
  void* y;                    /* (b, t, h, d) at + b*y_sb + t*y_st + h*HD + d, storage dtype */
  int64_t y_sb, y_st;
  /* mode 0, bf16 only: split of the key fields so that the window part can run before the
     consolidation chain has produced the slot snapshots.  part 0: all fields at once;
     part 1: sinks + window for every chunk (chunks 0 and 1 complete; chunks >= 2 leave their
     online-softmax state in `partial`); part 2: the slot field of chunks >= 2, merged with
     that state, then the readout.  partial: [B][H][n_q][HD + 4] floats. */
  int32_t part;
  float* partial;
  /* mode 0, bf16: only chunks [chunk_begin, chunk_end) (chunk_end == 0: to the last chunk), so that
     the slot field of early chunks can run while the chain still works on later steps */
  int32_t chunk_begin, chunk_end;
  /* mode 0, optional (NULL: not written): [B][H][n_q] fp32, every query's log-sum-exp (natural log)
     of its scaled, biased scores over all its keys -- the softmax normaliser the backward reuses */
  float* lse;
  /* mode 0, part 0, bf16, optional: the query heads straight from the q projection output, so that
     the q head preparation is done inside this kernel and q_rope, q_raw and eta are neither read
     nor needed (they may be NULL).  The values are those bolt3_heads computes (q RMSNorm, RoPE,
     tanh gate), bit for bit.  q_lin: element (b, t, c) at + (b*n_q + t)*q_lin_stride + c, query head
     h at columns h*HD..; qn_w: [HD] fp32 q RMSNorm weight, or NULL for none; rope_cs: the (cos, sin)
     table of positions 0..n_q-1 (b3_heads_args.rope_cs); gates: eta's pre-activation of head h at
     + (b*n_q + t)*gates_stride + gates_col + h.  Rows 16-byte aligned. */
  const void* q_lin;
  int64_t q_lin_stride;
  const float* qn_w;
  float qn_eps;
  const uint32_t* rope_cs;
  const void* gates;
  int64_t gates_stride;
  int32_t gates_col;
} b3_attn_args;

/*
 * Chunk attention: joint softmax over [sinks | attractor slots | causal window]
 * with GQA sharing, plus the M_res readout, for every chunk of a forward (mode 0)
 * or one step's queries (mode 1).
 * Replaces vsa_lm/config/bolt3.py:219-258 (forward chunk body) and :365-402
 * (Bolt3Decoder.step attention + readout).
 */
int bolt3_chunk_attn(const b3_attn_args* a, void* stream);

/*
 * Backward of a forward's chunk attention and M_res readout (bolt3_chunk_attn, mode 0): given
 * dy, the gradient of the attention + readout output, the gradients with respect to the roped
 * queries, the un-roped queries (readout), eta, every key field (window keys and values, sinks,
 * the slot snapshots of every step), the slot bias, M_res of every step, res_norm's weight and
 * gamma, from the forward's own row log-sum-exps (b3_attn_args.lse).  fp32 storage: fp32
 * arithmetic; bf16 storage: MFMA products of bf16 operands with fp32 accumulation.  The row
 * gradients of storage-dtype tensors come in the storage dtype, the rest in fp32.  Every output
 * element has one writer; d_q_raw, d_eta, d_res_w, d_gamma, d_bias and the sink gradients must be
 * zero-filled by the caller (chunks without a readout or without those fields leave them
 * untouched).
 * Replaces the autograd backward of vsa_lm/config/bolt3.py:219-256 (softmax over
 * [sinks | slots | window], the value read, the readout eta * res_norm(normalize(q) M (1-g)/sqrt(HD))).
 */
typedef struct {
  int32_t dtype, B, T, H, HKV, HD, S, C, n_sinks;
  int32_t n_chunks;           /* ceil(T / C) */
  int32_t n_qtiles;           /* ceil(C / 32): query tiles per chunk */
  int32_t n_steps;            /* consolidation steps of the forward: chunk c >= 2 reads step c - 2 */
  int32_t score_round;        /* as in b3_attn_args (1 for the forward) */
  const void* q_rope;         /* (b, h, t, d) at + b*q_sb + h*q_sh + t*HD + d, storage dtype */
  const void* q_raw;
  int64_t q_sb, q_sh;
  const void* win_k;          /* (b, hkv, t, d) at + b*w_sb + hkv*w_sh + t*HD + d: roped keys of every token */
  const void* win_v;
  int64_t w_sb, w_sh;
  const void* slot_k;         /* [step][B*HKV][S][HD] roped slot keys, as the forward's snapshots */
  const void* slot_v;
  const float* slot_bias;     /* [step][B*HKV][S] */
  int64_t slot_step;          /* elements between steps of slot_k / slot_v */
  const float* m_res;         /* [step][B*HKV] blocks of HD*HD floats, layout as b3_attn_args.m_split */
  int64_t m_step;
  int32_t m_split;
  const float* eta;           /* (b, h, t) at + b*e_sb + h*e_sh + t */
  int64_t e_sb, e_sh;
  const float* gamma;         /* [HKV] */
  const float* res_w;         /* [HD] */
  float eps;
  const void* y;              /* forward output before o_proj, (b, t, h, d) at + b*y_sb + t*y_st + h*HD + d */
  int64_t y_sb, y_st;
  const void* dy;             /* its gradient in the storage dtype, (b, t, h, d) at + b*dy_sb + t*dy_st + h*HD + d */
  int64_t dy_sb, dy_st;
  float* d_rows;              /* [B][H][T] written: sum over d of dy * attention output */
  const float* lse;           /* [B][H][T] every query row's log-sum-exp (natural log) as the forward wrote it
                                 (b3_attn_args.lse of the bolt3_chunk_attn call that made y) */
  /* d_q_rope, d_q_raw and the d_k_* / d_v_* row gradients are in the storage dtype (the
     gradients of storage-dtype tensors); the rest is fp32 */
  void* d_q_rope;             /* [B][H][T][HD] */
  void* d_q_raw;              /* [B][H][T][HD] (readout part; rows of chunks without a readout are
                                 not written) */
  float* d_eta;               /* [B][H][T] (rows of chunks without a readout are not written) */
  float* d_m;                 /* [step][B*HKV][HD][HD]: gradient of M_res of step c - 2 from chunk c */
  float* d_res_w;             /* [B*HKV][n_chunks][HD] partial sums (zero-filled) */
  float* d_gamma;             /* [B*HKV][n_chunks] partial sums (zero-filled) */
  float* d_bias;              /* [step][B*H][n_qtiles][S] partial sums of the slot bias gradient */
  void* d_k_own;              /* [B][HKV][T][HD]: keys of chunk c from chunk c's queries */
  void* d_v_own;
  void* d_k_next;             /* [B][HKV][T][HD]: keys of chunk c from chunk c+1's queries (rows of the
                                 last chunk are not written) */
  void* d_v_next;
  float* d_slot_k;            /* [step][B*HKV][S][HD] */
  float* d_slot_v;
  float* d_sink_k;            /* [n_chunks][B*HKV][n_sinks][HD] (chunks 0 and 1 are not written) */
  float* d_sink_v;
  int32_t part;               /* 0: everything; 1: the readout kernels only (d_m, d_q_raw, d_eta, d_res_w,
                                 d_gamma, d_rows); 2: the attention kernels only, after a part-1 call
                                 with the same arguments (they read d_rows) */
  void* rd_rows;              /* bf16 storage, parts 0 and 1 with a readout: [B][H][T][HD] bf16 scratch
                                 rows (du / |q_raw| of the readout's rows, written by its row kernel and
                                 read by its dM kernel).  May be d_q_rope: with part 0, or part 2 after
                                 part 1, the attention kernels overwrite every row of it afterwards.
                                 Unused (may be NULL) for fp32 storage or part 2. */
} b3_attn_bwd_args;
int bolt3_attn_bwd(const b3_attn_bwd_args* a, void* stream);

typedef struct {
  int32_t dtype, B, H, HKV, HD, S;
  const void* lin;            /* [B][lin_row_stride] packed projection row of the new token */
  int64_t lin_row_stride;
  const float* qn_w;          /* [HD] fp32 q/k RMSNorm weights or NULL */
  const float* kn_w;
  int32_t has_qk_norm;
  float eps;                  /* q/k norm and res_norm epsilon */
  const float* inv_freq;
  int32_t pos;                /* position of the new token */
  void* win_kr;               /* window ring (b, hkv, n, d) at + b*w_sb + hkv*w_sh + n*HD + d */
  void* win_kp;
  void* win_v;
  int64_t w_sb, w_sh;
  float* win_beta;            /* (b, hkv, n) at + b*wb_sb + hkv*wb_sh + n */
  int64_t wb_sb, wb_sh;
  float* win_pos;             /* fp32 [n] */
  int32_t a_start, a_len;     /* older window segment */
  int32_t b_start, b_len;     /* current segment before the new token; new token goes to b_start + b_len */
  const void* sink_k;
  const void* sink_v;
  int64_t s_sb, s_sh;
  int32_t n_sink_keys;
  const void* slot_k;         /* [bh][S][HD] roped slot keys */
  const void* slot_v;
  const float* slot_bias;     /* [bh][S] */
  int32_t has_slots;
  const float* m_res;         /* [bh][HD][HD] */
  const float* gamma;
  const float* res_w;
  void* y;                    /* [B][H*HD] storage dtype */
  float* work;                /* scratch of >= bolt3_decode_workspace_bytes(B, H, HKV, HD) bytes */
  int64_t work_bytes;
  /* Graph-stable steps (bf16 bolt3_decode_layer only): when step_desc is set the kernels read
     pos, a_start, a_len, b_start, b_len, n_sink_keys, has_slots from step_desc[0..6] (device
     memory, advanced by bolt3_step_advance) instead of the fields above, and clamp every window
     index into [0, ring_cap), the tokens per (b, hkv) of win_*.  NULL: the fields above. */
  const int32_t* step_desc;
  int32_t ring_cap;
} b3_decode_args;

/*
 * Softmax-anchor mode of the one-token step (bf16 bolt3_decode_layer only): win_kr == NULL and
 * win_beta == NULL, no sinks, no slots, m_res == NULL.  The projection row then holds only
 * q | k | v; the roped key and the value are appended at b_start + b_len of win_kp / win_v (the
 * layer's key/value cache) and the output is plain causal softmax attention over
 * [a_start, a_start + a_len) and the new token, with any number of keys.  Replaces the anchor
 * branch of vsa_lm/config/bolt3.py:426-445 for t_s == 1 (StaticKV append + SDPA), projections
 * and o_proj included.
 *
 * One-token decode step of a Bolt-3 layer: head prep for the new token, append to
 * the window ring, attention over sinks + slots + window in fp32 scores, M_res
 * readout.  Three kernels on the stream: the new token's head preparation, the key
 * ranges of every (batch, kv head) in parallel plus the readout, then the merge of
 * the ranges.
 * Replaces vsa_lm/config/bolt3.py:346-402 for t_s == 1.
 */
int bolt3_decode(const b3_decode_args* a, void* stream);
/*
 * Adds (d_pos, d_a_start, d_a_len, d_b_start, d_b_len) to step_desc[0..4]: the device-side
 * advance of a graph-captured decode step (one workgroup of one wavefront).  No counterpart in
 * the reference (its step has no graph, vsa_lm/config/bolt3.py:287-288).
 */
int bolt3_step_advance(int32_t* step_desc, int32_t d_pos, int32_t d_a_start, int32_t d_a_len, int32_t d_b_start,
                       int32_t d_b_len, void* stream);

/* Workspace of bolt3_decode: partial softmax state of the key ranges and the readout per (batch, kv head). */
int64_t bolt3_decode_workspace_bytes(int32_t B, int32_t H, int32_t HKV, int32_t HD);

/*
 * A whole one-token decode layer step in bf16: the packed input projection
 * x . W_in^T + b_in (W_in rows q | k | v | beta | eta, zero rows padding to n_in), the
 * bolt3_decode step on that row, then out = y . W_out^T + b_out.  The projections stream
 * each weight once (workgroups of 128 weight rows x 512 columns of K, x staged in LDS) and
 * leave fp32 partial products per K chunk in proj_work, added in order and rounded once by
 * their consumer.
 * Replaces vsa_lm/config/bolt3.py:346-402 for t_s == 1 together with the q/k/v/beta/eta
 * projections it calls (:59-66, :349) and o_proj (:400-402).
 */
typedef struct {
  b3_decode_args dec;         /* dec.lin unused (the row comes from the projection); dec.lin_row_stride = n_in;
                                 dec.y: [B][H*HD] attention output, written */
  const void* x;              /* [B][x_row_stride] layer input rows, 16-byte aligned */
  int64_t x_row_stride;       /* multiple of 8 */
  int32_t d_model;            /* columns of x = columns of W_in, multiple of 32 */
  const void* w_in;           /* [n_in][d_model] row-major */
  const void* b_in;           /* [n_in] or NULL */
  int32_t n_in;               /* = dec.lin_row_stride, multiple of 16 */
  const void* w_out;          /* [n_out][H*HD] row-major */
  const void* b_out;          /* [n_out] or NULL */
  int32_t n_out;              /* multiple of 16 */
  void* out;                  /* [B][out_row_stride] */
  int64_t out_row_stride;     /* multiple of 4 */
  float* proj_work;           /* >= bolt3_decode_layer_workspace_bytes(B, d_model, n_in, H*HD, n_out) bytes */
  int64_t proj_work_bytes;
} b3_decode_layer_args;
int bolt3_decode_layer(const b3_decode_layer_args* a, void* stream);
/* Workspace of bolt3_decode_layer's projections (besides dec.work): the fp32 partial products. */
int64_t bolt3_decode_layer_workspace_bytes(int32_t B, int32_t d_model, int32_t n_in, int32_t hd_total, int32_t n_out);

/*
 * RMSNorm of rows: y = (x * rsqrt(mean(x^2) + eps)) * w with an fp32 statistic, each product
 * rounded in fp32 and the result cast to the storage dtype (x's) once.  For the layers around
 * the Bolt-3 path in a hybrid stack (block norms, final norm, the softmax layers' q/k norms).
 * Replaces vsa_lm/surgery.py:48-52 (LlamaRMSNorm.forward) on the device.
 */
typedef struct {
  int32_t dtype;              /* of x and y */
  int64_t rows;
  int32_t dim;                /* multiple of 8 */
  const void* x;              /* [rows][x_row_stride], 16-byte aligned rows */
  int64_t x_row_stride;
  const void* w;              /* [dim] */
  int32_t w_dtype;
  void* y;                    /* [rows][y_row_stride] */
  int64_t y_row_stride;
  float eps;
} b3_rms_norm_args;
int bolt3_rms_norm(const b3_rms_norm_args* a, void* stream);

/*
 * Backward of the consolidation chain (bf16 or fp32 storage, HD in {64, 128}, S == 128, at most
 * 128 tokens per step), from the forward chain's decision log and per-step snapshots.  The decisions are
 * constants (the reference takes them under no_grad, vsa_lm/config/bolt3.py:98-112, :121-135,
 * :165-180); the gradient flows through the copies and mass-weighted means that fill, merge and
 * evict the slots (:121-155, :182-191) and through the Gershgorin-safe delta rule
 * M <- gamma M + Khat^T diag(bsafe) (V - Khat M) (:154-162).  Four kernels on the stream: per
 * (step, bh) the tokens' 1/|k|, Gershgorin row sums and delta weights; per (bh, 16 features)
 * the slot-gradient recursion with its token scatters; per (bh, 32 columns of M) the
 * M_res-gradient recursion G_i = dM_i + (gamma I - Khat^T diag(bsafe) Khat) G_{i+1}; per
 * (step, bh) the delta rule's token gradients.  Replaces the autograd of :121-166 and :182-191
 * for Bolt3Attn.forward's chain (:262-273).
 */
typedef struct {
  int32_t dtype, B, HKV, HD, S, T;
  int32_t n_steps, off0, len0, step_stride, step_len;   /* the forward chain's step layout (empty start) */
  const void* kr;             /* [B*HKV][T][HD] un-roped keys (storage dtype) */
  const void* v;              /* [B*HKV][T][HD] values (storage dtype) */
  const float* beta;          /* [B*HKV][T] delta-rule gates */
  const float* log;           /* [n_steps][B*HKV][B3_LOG_ROWS][B3_LOG_COLS] the forward's decision log */
  const float* snap_mass;     /* [n_steps][B*HKV][S] slot mass after every step */
  const float* snap_pm;       /* [n_steps][B*HKV][S] slot mean position after every step */
  const float* snap_m;        /* [n_steps][B*HKV] blocks of HD*HD floats: bf16 storage M^T as bf16 hi then
                                 bf16 lo, fp32 storage M[c][d] (the forward chain's snapshots) */
  const float* gamma;         /* [HKV] */
  const float* inv_freq;      /* [HD/2] */
  const float* d_slot_k;      /* [n_steps][B*HKV][S][HD] gradient of the roped slot keys the attention read */
  const float* d_slot_v;      /* [n_steps][B*HKV][S][HD] */
  const float* d_m;           /* [n_steps][B*HKV][HD][HD] gradient of M_res after every step, M[c][d] */
  float* d_kr;                /* added to: [B*HKV][T][HD] gradient of the un-roped keys */
  float* d_v;                 /* added to: [B*HKV][T][HD] */
  float* d_beta;              /* added to: [B*HKV][T] */
  float* d_gamma;             /* out: [n_steps][B*HKV][HD/32] partial sums of dL/dgamma */
  void* work;                 /* >= bolt3_chain_bwd_workspace_bytes(...) bytes */
  int64_t work_bytes;
  int32_t kernels;            /* which of the four kernels this call launches, in their order: a mask of
                                 B3_CBWD_* bits, 0 = all.  Calls that split them keep the order (token
                                 statistics before the M_res recursion and the token gradients, both
                                 recursions before the token gradients) and the same arguments and
                                 workspace; the two recursions touch disjoint data and may run on
                                 different streams.  The statistics and the M_res recursion read d_m
                                 only, the slot recursion d_slot_k / d_slot_v only */
  uint32_t* started;          /* optional (NULL to skip): each workgroup of the M_res and slot recursions
                                 that this call launches adds 1 when it begins (B*HKV*HD/32 and
                                 B*HKV*HD/16 of them), for bolt3_wait_count */
} b3_chain_bwd_args;
#define B3_CBWD_STATS 1
#define B3_CBWD_M_REC 2
#define B3_CBWD_SLOT_REC 4
#define B3_CBWD_TOK_GRAD 8
#define B3_CBWD_ALL 15
int bolt3_chain_bwd(const b3_chain_bwd_args* a, void* stream);
int64_t bolt3_chain_bwd_workspace_bytes(int32_t B, int32_t HKV, int32_t HD, int32_t n_steps);

/*
 * Backward of Bolt3Attn's head preparation, one pass per token row: the gradients of the roped
 * queries and keys through the transpose of their RoPE (vsa_lm/config/bolt3.py:214-215,
 * vsa_lm/surgery.py:86-93), plus the readout's gradient of the un-roped queries and the chain's
 * of the un-roped keys and values; the sinks' and the next chunk's key / value gradients; the q / k
 * RMSNorm backward (:203-206, vsa_lm/surgery.py:48-52) with per-block partial sums of the norm
 * weights' gradients; the gates' derivatives beta = sigmoid(.), eta = tanh(.) (:198-199).  Writes
 * dz, the gradient of the packed projection output [q | k | v | beta | eta | zero pad] per row
 * (storage dtype), which the projection-gradient products read.  HD in {64, 128}.
 */
typedef struct {
  int32_t dtype, B, T, H, HKV, HD, n_sinks, n_chunks;
  /* the six row gradients of bolt3_attn_bwd, in the storage dtype */
  const void* d_q_raw;        /* [B][H][T][HD] gradient of the un-roped queries (readout) */
  const void* d_q_rope;       /* [B][H][T][HD] gradient of the roped queries (attention) */
  const void* d_k_own;        /* [B][HKV][T][HD] gradient of the roped keys as their own chunk's keys */
  const void* d_k_next;       /* [B][HKV][T][HD] ... as the next chunk's keys */
  const void* d_v_own;
  const void* d_v_next;
  const float* d_sink_k;      /* [n_chunks][B*HKV][n_sinks][HD] or NULL: the sinks' roped-key gradients */
  const float* d_sink_v;
  const float* d_k_chain;     /* [B*HKV][T][HD] or NULL: the chain's gradient of the un-roped keys */
  const float* d_v_chain;     /* [B*HKV][T][HD] or NULL */
  const float* d_beta;        /* [B*HKV][T] or NULL */
  const float* d_eta;         /* [B][H][T] */
  const float* beta;          /* [B][HKV][T] gate values */
  const float* eta;           /* [B][H][T] */
  const void* lin_q;          /* [B*T][lin_q_row_stride] pre-norm q projection (storage dtype) */
  int64_t lin_q_row_stride;
  const void* lin_k;          /* [B*T][lin_k_row_stride] pre-norm k projection */
  int64_t lin_k_row_stride;
  const float* qn_w;          /* [HD] */
  const float* kn_w;
  int32_t has_qk_norm;
  float q_eps, k_eps;
  const float* inv_freq;      /* [HD/2] */
  void* dz;                   /* out: [B*T][dz_row_stride] storage dtype; dz_row_stride and the lin row
                                 strides are multiples of 4 elements (rows move as 4-element vectors) */
  int64_t dz_row_stride;
  int32_t dz_cols;            /* >= (H + 2 HKV) HD + HKV + H; the columns past those are zeroed */
  float* d_qn_w;              /* out: [bolt3_heads_bwd_blocks(B, T)][HD] partial sums (has_qk_norm) */
  float* d_kn_w;
  int32_t parts;              /* 0: everything; 1: the query heads, the eta columns and d_qn_w (reads
                                 neither the chain's nor the keys' gradients); 2: the key / value heads,
                                 the beta columns, the pad and d_kn_w.  Parts 1 and 2 write disjoint
                                 columns and may run on different streams */
} b3_heads_bwd_args;
int bolt3_heads_bwd(const b3_heads_bwd_args* a, void* stream);
int32_t bolt3_heads_bwd_blocks(int32_t B, int32_t T);

/* Library identification: returns a static string (build flags, gfx target). */
const char* bolt3_version(void);

#ifdef __cplusplus
}
#endif

#endif /* BOLT3_AMD_H */
