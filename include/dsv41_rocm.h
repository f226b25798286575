/*
 * dsv41_rocm.h — C ABI of libdsv41hip.so, the MI355X (gfx950) implementation of
 * Tiny-DSV41's token-sampling step and fused selected-token log-prob head.
 *
 * Plain C: pointers, sizes and PODs only. Every device pointer is a HIP device
 * address owned by the caller; the library never allocates or frees device
 * memory, never synchronises the stream, and launches only on `stream`.
 *
 * Return codes: 0 on success, a negative DSV41_E_* code before any launch on a
 * bad argument. dsv41_last_error() then holds a thread-local message whose text
 * mirrors the reference's ValueError messages where one exists.
 *
 * Reference interfaces replaced (paths relative to the Tiny-DSV41 tree):
 *   dsv41_sampler_run  <- dsv41_train/rl/rollout.py:144-150 (log_softmax(logits/T),
 *                         isfinite check, multinomial draw, behaviour log-prob),
 *                         extended with the vLLM SamplingParams knobs named at
 *                         rollout_manager/backends/vllm_actor.py:178-185.
 *   dsv41_logprob_run  <- dsv41_train/models/dsv4/model.py:679-684 (_token_log_probs),
 *                         dsv41_train/rl/native_lora.py:80-82 (_score_targets),
 *                         plus the Token-TIS weight of dsv41_train/rl/algorithm.py:293-299.
 *   dsv41_sampler_shard_run + dsv41_sampler_merge_run <- the same lines for logits whose
 *                         vocabulary is split over tensor-parallel GPUs (top-k draws).
 *   dsv41_sampler_full_state_run + dsv41_sampler_full_draw_run + dsv41_sampler_full_finish_run
 *                      <- the same lines, the full-vocabulary draw of rollout.py:144-148
 *                         (training's default, rollout_manager/training.py:74-81), over
 *                         split vocabularies.
 *   dsv41_grpo_run     <- dsv41_train/rl/algorithm.py:169-246 (grpo_loss).
 *   dsv41_token_tis_run <- dsv41_train/rl/algorithm.py:249-346 (decoupled_token_tis_loss)
 *                         with the metric pooling of dsv41_train/rl/distributed_grpo.py:197-222.
 *   dsv41_logprob_grad_run <- the autograd backward of that expression as the learner
 *                         differentiates it (dsv41_train/rl/distributed_grpo.py:352-375 over
 *                         native_lora.py:120-122 / model.py:735-738): the gradient with
 *                         respect to the lm_head output, in that output's dtype (bf16).
 */
#ifndef DSV41_ROCM_H
#define DSV41_ROCM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSV41_ABI_VERSION 6

/* Element types of logits / activations. */
#define DSV41_DTYPE_F32 0
#define DSV41_DTYPE_BF16 1

/* Error codes (negative returns). */
#define DSV41_OK 0
#define DSV41_E_INVALID (-1)     /* bad shape, stride, pointer or parameter value   */
#define DSV41_E_UNSUPPORTED (-2) /* valid request beyond on-chip limits of a kernel  */
#define DSV41_E_WORKSPACE (-3)   /* workspace missing or smaller than required       */
#define DSV41_E_HIP (-4)         /* a HIP runtime call failed                        */
#define DSV41_E_ABI (-5)         /* descriptor struct_size does not match this build  */

/* Per-row / per-token status bits written to out_status (0 = clean). */
#define DSV41_STATUS_NONFINITE 1   /* a processed logit / result was NaN or +-inf      */
#define DSV41_STATUS_BAD_HISTORY 2 /* a history id was >= vocab (id ignored); history  */
                                   /* is read only when a penalty is active             */
#define DSV41_STATUS_BAD_UNIFORM 4 /* uniform outside [0, 1) (row drawn with u = 0)    */
#define DSV41_STATUS_RATIO_ZERO 8  /* Token-TIS raw weight exp(old - behaviour) == 0   */
#define DSV41_STATUS_BAD_TARGET 16 /* a replay id was outside [0, vocab) (lp = NaN)    */
#define DSV41_STATUS_BAD_SLICES 32 /* full-vocabulary draw over slices: the gathered    */
                                   /* masses place the target in no slice's own masses  */
                                   /* (states, masses and draw step from other inputs); */
                                   /* id -1, lp NaN                                     */

/*
 * Row sampler.  For each row r of logits[rows, vocab]:
 *   x = float(logit); for ids in the row's history (c = count, see history_prompt_lens):
 *     x = x > 0 ? x / repetition_penalty : x * repetition_penalty;
 *     x = x - frequency_penalty * c;  if (c > 0) x = x - presence_penalty;
 *   z = x / temperature;
 *   min-p  (min_p > 0): keep z_i - z_max >= log(min_p) (fp64);
 *   top-k  (top_k > 0): keep the first top_k of the survivors in (z desc, index asc);
 *   top-p  (top_p < 1): keep the shortest prefix of that order whose 2^-43 fixed-point
 *                       mass reaches ceil(top_p * total);
 *   draw: inverse CDF in vocabulary order over the kept set against uniforms[r], on the
 *         2^-43 fixed-point masses floor(2^43 exp(z_i - z_max)) (exp evaluated by a fixed
 *         sequence of fp32 operations, identical on every device and in the oracle): the
 *         first token whose cumulative mass exceeds (total * floor(u * 2^32)) >> 32, exact
 *         in integers (greedy != 0: first index of max z instead);
 *   out_logprob = z_tok - log(sum_kept exp(z)), out_kept = kept-set size.
 * history[r * history_row_stride + j], j < (history_lens ? history_lens[r] : hist_len);
 * negative ids are padding and ignored.  With history_prompt_lens, the first
 * history_prompt_lens[r] entries of row r are the prompt's ids and the rest the generated
 * ones, and the penalties follow vLLM's rule: the repetition penalty applies to ids of the
 * prompt or the output, the frequency and presence penalties count the output only (c is the
 * id's count among the generated entries; presence applies when c > 0).  Without it every
 * entry counts as generated.
 */
typedef struct dsv41_sampler_desc {
  uint32_t struct_size; /* = sizeof(dsv41_sampler_desc) */
  int32_t rows;
  int32_t vocab;
  int32_t logits_dtype;        /* DSV41_DTYPE_F32 or DSV41_DTYPE_BF16 */
  int64_t logits_row_stride;   /* in elements */
  const void* logits;          /* [rows, vocab] */
  const int64_t* history;      /* [rows, history_row_stride] or NULL */
  int64_t history_row_stride;  /* in elements */
  int32_t hist_len;            /* ids per row when history_lens == NULL */
  const int32_t* history_lens; /* [rows] or NULL */
  const float* uniforms;       /* [rows]; may be NULL only when greedy != 0 */
  float temperature;           /* finite, > 0 */
  float repetition_penalty;    /* finite, > 0; 1 = off */
  float presence_penalty;      /* finite; 0 = off */
  float frequency_penalty;     /* finite; 0 = off */
  int32_t top_k;               /* 0 = off */
  float top_p;                 /* (0, 1]; 1 = off */
  float min_p;                 /* [0, 1]; 0 = off */
  int32_t greedy;              /* nonzero: argmax instead of the draw */
  int64_t* out_ids;            /* [rows] */
  float* out_logprob;          /* [rows], or NULL: no log-probs (required with replay_ids); a
                                  greedy draw without truncation then forms no masses, only
                                  each row's first maximum */
  int32_t* out_kept;           /* [rows] or NULL */
  int32_t* out_status;         /* [rows] */
  /* Exponential-race draw (no truncation only): token = argmax_i p_i / exponentials[r, i]
   * with p = exp(log_softmax(z)) in fp32, first index on ties: torch.multinomial(p, 1) as
   * the CPU computes it (exponential_ then argmax(p / E)) when fed the same variates.
   * NULL: inverse CDF against uniforms. */
  const float* exponentials;       /* [rows, exponentials_row_stride] or NULL */
  int64_t exponentials_row_stride; /* in elements, >= vocab */
  /* Replay (no truncation only): no draw; out_logprob[r] = the processed log-prob of token
   * replay_ids[r], bit for bit the value a draw of that token reports on the same logits and
   * knobs (behaviour log-probs replayed exactly, rl/qwen_policy.py:156-190); out_ids echoes
   * the id.  uniforms may be NULL. */
  const int64_t* replay_ids;       /* [rows] or NULL */
  const int32_t* history_prompt_lens; /* [rows] or NULL: leading history entries of the prompt */
} dsv41_sampler_desc;

/*
 * One GPU's slice of vocabulary-sharded logits (a tensor-parallel head): `sampler` describes
 * the slice [rows, vocab] holding the ids [vocab_offset, vocab_offset + vocab) of a vocab_size
 * vocabulary, with the row knobs of the whole batch (1 <= top_k <= 2048).
 * History ids are global; sampler->uniforms, out_ids, out_logprob and out_kept are unused.
 * For each row the slice emits its exact local top_k under the local min-p bound: at most
 * top_k candidate keys, each
 *   key = (okey(z) << 32) | (0xFFFFFFFF - global id),
 *   okey(z) = bits(z) | 0x80000000 for z >= 0, ~bits(z) for z < 0 (-0 as +0),
 * so that keys order as (z descending, id ascending).  The row's local maximum is at most
 * its global one, so the union of the slices' lists holds the row's kept set, and
 * dsv41_sampler_merge_run finishes every row exactly as dsv41_sampler_run would.  The lists
 * (up to 8 * top_k bytes per row and slice), counts and status bits are the wire format.
 */
typedef struct dsv41_sampler_shard_desc {
  uint32_t struct_size;              /* = sizeof(dsv41_sampler_shard_desc) */
  int32_t max_candidates;            /* keys per row in out_keys, >= sampler->top_k */
  const dsv41_sampler_desc* sampler;
  int64_t vocab_offset;              /* global id of the slice's first column */
  int64_t vocab_size;                /* the whole vocabulary; larger history ids flag the row */
  uint64_t* out_keys;                /* [rows, max_candidates] */
  int32_t* out_counts;               /* [rows] */
  int32_t* out_status;               /* [rows] DSV41_STATUS_* bits seen by this slice */
} dsv41_sampler_shard_desc;

/*
 * Full-vocabulary draws (no top-k, top-p or min-p) over vocabulary slices, in steps with one
 * all-gather after each:
 *   1. dsv41_sampler_full_state_run: each slice streams its columns once (penalties from the
 *      global history ids, then / T) and writes one dsv41_full_state per row;
 *   2. inverse CDF only: with the states of all slices gathered ([n_shards, rows], slices in
 *      vocabulary order), dsv41_sampler_full_mass_run forms the row's maximum M and writes
 *      the slice's exact fixed-point mass sum_i floor(2^43 exp(z_i - M)) (u64) per row;
 *   3. dsv41_sampler_full_draw_run, with the states (and for the inverse CDF the masses)
 *      gathered.  Inverse CDF: the target is (S * floor(u * 2^32)) >> 32 over the integer
 *      total S of the masses; the slice whose masses hold it re-reads its columns and picks
 *      the token exactly as dsv41_sampler_run would, the others report none.  Exponential
 *      race: every slice reports its best p / E over its columns with
 *      p = exp(z - (M + log S')) in fp32, S' = sum_s mass_s * exp(max_z_s - M) over the
 *      states in slice order (fp64), first id on ties;
 *   4. with the picks gathered, dsv41_sampler_full_finish_run writes ids, log-probs
 *      lp = (z_tok - M) - log S', kept = vocab_size and status bits, as dsv41_sampler_run
 *      does (greedy needs only the states: the first slice holding M gives its argmax).
 * The states (32 bytes), masses (8 bytes) and picks (16 bytes) per row and slice are the
 * wire format.
 */
typedef struct dsv41_full_state {
  float max_z;      /* the slice's largest processed logit; -inf when it has none */
  int32_t status;   /* DSV41_STATUS_* bits seen by this slice */
  double mass;      /* sum over the slice of exp(z - max_z): its exact fixed-point masses
                       against max_z (integers, as dsv41_sampler_run forms them) times 2^-43 */
  int64_t argmax;   /* global id of the slice's first largest logit */
  int64_t reserved;
} dsv41_full_state;

typedef struct dsv41_full_pick {
  int64_t id;       /* global id chosen by this slice, or -1 */
  float z;          /* its processed logit */
  float ratio;      /* exponential race: its p / E */
} dsv41_full_pick;

typedef struct dsv41_sampler_full_shard_desc {
  uint32_t struct_size;              /* = sizeof(dsv41_sampler_full_shard_desc) */
  int32_t n_shards;                  /* draw step: slices in `states` */
  const dsv41_sampler_desc* sampler; /* the slice [rows, vocab] holding ids [vocab_offset,
                                        vocab_offset + vocab); knobs without truncation;
                                        draw step: uniforms, or exponentials over the slice's
                                        columns (race); out_* unused */
  int64_t vocab_offset;              /* global id of the slice's first column */
  int64_t vocab_size;                /* the whole vocabulary; larger history ids flag the row */
  int32_t shard_index;               /* draw step: this slice's position in `states` */
  int32_t reserved;
  const dsv41_full_state* states;    /* mass and draw steps: [n_shards, rows], gathered */
  dsv41_full_state* out_states;      /* state step: [rows] */
  dsv41_full_pick* out_picks;        /* draw step: [rows] */
  const uint64_t* masses;            /* inverse-CDF draw step: [n_shards, rows], gathered */
  uint64_t* out_masses;              /* mass step: [rows] */
} dsv41_sampler_full_shard_desc;

#define DSV41_FULL_DRAW_CDF 0     /* inverse CDF against uniforms */
#define DSV41_FULL_DRAW_RACE 1    /* exponential race */
#define DSV41_FULL_DRAW_GREEDY 2  /* first largest logit (no draw step) */

typedef struct dsv41_sampler_full_finish_desc {
  uint32_t struct_size;            /* = sizeof(dsv41_sampler_full_finish_desc) */
  int32_t rows;
  int32_t n_shards;
  int32_t draw;                    /* DSV41_FULL_DRAW_* */
  const dsv41_full_state* states;  /* [n_shards, rows] */
  const dsv41_full_pick* picks;    /* [n_shards, rows]; unused for greedy */
  const float* uniforms;           /* inverse CDF: [rows], checked to lie in [0, 1) */
  int64_t vocab_size;
  int64_t* out_ids;                /* [rows] */
  float* out_logprob;              /* [rows] or NULL */
  int32_t* out_kept;               /* [rows] or NULL */
  int32_t* out_status;             /* [rows] */
} dsv41_sampler_full_finish_desc;

/* Finishes a sharded batch from the gathered lists of all slices. */
typedef struct dsv41_sampler_merge_desc {
  uint32_t struct_size;    /* = sizeof(dsv41_sampler_merge_desc) */
  int32_t rows;
  int32_t n_shards;
  int32_t max_candidates;  /* keys per row and slice in `keys` */
  const uint64_t* keys;    /* [n_shards, rows, max_candidates], each list in any order; lists
                              sorted descending, as dsv41_sampler_shard_run leaves them, take
                              a faster merge when top_k <= 64 */
  const int32_t* counts;   /* [n_shards, rows] */
  const int32_t* status;   /* [n_shards, rows] */
  const float* uniforms;   /* [rows]; may be NULL only when greedy != 0 */
  int32_t top_k;           /* the knobs of the shard launches */
  float top_p;
  float min_p;
  int32_t greedy;
  int64_t* out_ids;        /* [rows] */
  float* out_logprob;      /* [rows] or NULL */
  int32_t* out_kept;       /* [rows] or NULL */
  int32_t* out_status;     /* [rows]: the OR of the slices' bits and the uniform check */
} dsv41_sampler_merge_desc;

/*
 * Fused selected-token log-prob.  logits = x[N,H] @ w[V,H]^T in fp32 (never stored),
 * z = logits / temperature; for each token n:
 *   out_logprob[n] = z[n, targets[n]] - logsumexp(z[n, :])
 *   out_entropy[n] = logsumexp(z[n, :]) - sum_v softmax(z[n])_v * z[n, v]
 *   out_ratio[n]   = float(min(is_cap, exp(double(float(out_logprob[n] - behavior[n])))))
 *                    when behavior != NULL (Token-TIS weight, algorithm.py:293-299).
 */
typedef struct dsv41_logprob_desc {
  uint32_t struct_size; /* = sizeof(dsv41_logprob_desc) */
  int32_t n_tokens;
  int32_t hidden;
  int32_t vocab;
  const void* x;          /* bf16 [N, H] */
  int64_t x_row_stride;   /* in elements, multiple of 8 */
  const void* w;          /* bf16 [V, H] (nn.Linear weight layout) */
  int64_t w_row_stride;   /* in elements, multiple of 8 */
  const int64_t* targets; /* [N], each in [0, V) */
  float temperature;      /* finite, > 0 */
  const float* behavior;  /* [N] or NULL */
  float is_cap;           /* finite, > 0 (used when behavior != NULL) */
  float* out_logprob;     /* [N] */
  float* out_entropy;     /* [N] or NULL */
  float* out_ratio;       /* [N] or NULL; requires behavior */
  int32_t* out_status;    /* [N] or NULL */
  float* out_lse;         /* [N] or NULL: logsumexp(z[n, :]), kept for the backward */
} dsv41_logprob_desc;

/*
 * One GPU's slice of a vocabulary-sharded head (tensor-parallel lm_head): w holds the head's
 * rows [vocab_offset, vocab_offset + vocab).  For each token, out_state[n] (16 bytes, the
 * wire format of the sharded path) = (m, s, a, z_t) over this slice:
 *   m = max_v z[n, v],  s = sum_v exp(z[n, v] - m),  a = sum_v exp(z[n, v] - m) * z[n, v],
 *   z_t = z[n, targets[n]] when this slice holds targets[n], -inf otherwise.
 * The states of all slices, gathered ([n_shards, N, 4]), combine exactly into the
 * unsharded result with dsv41_logprob_combine_run.
 */
typedef struct dsv41_logprob_shard_desc {
  uint32_t struct_size; /* = sizeof(dsv41_logprob_shard_desc) */
  int32_t n_tokens;
  int32_t hidden;
  int32_t vocab;          /* rows of this slice */
  const void* x;          /* bf16 [N, H] */
  int64_t x_row_stride;
  const void* w;          /* bf16 [vocab, H]: this slice's rows */
  int64_t w_row_stride;
  const int64_t* targets; /* [N], global ids */
  int64_t vocab_offset;   /* global id of w's first row */
  float temperature;
  float* out_state;       /* [N, 4] fp32 */
} dsv41_logprob_shard_desc;

/* Combines gathered shard states into the outputs of dsv41_logprob_run. */
typedef struct dsv41_logprob_combine_desc {
  uint32_t struct_size; /* = sizeof(dsv41_logprob_combine_desc) */
  int32_t n_tokens;
  int32_t n_shards;
  const float* states;    /* [n_shards, N, 4], 16-byte aligned */
  const float* behavior;  /* [N] or NULL */
  float is_cap;
  float* out_logprob;     /* [N] */
  float* out_entropy;     /* [N] or NULL */
  float* out_ratio;       /* [N] or NULL; requires behavior */
  int32_t* out_status;    /* [N] or NULL */
  float* out_lse;         /* [N] or NULL */
} dsv41_logprob_combine_desc;

/*
 * Gradient of a loss L(out_logprob, out_entropy) with respect to the logits, for the
 * vocabulary rows [vocab_begin, vocab_end):
 *   p = softmax(z[n]),  z = logits / temperature,
 *   dL/dz[n, v] = grad_logprob[n] * ([v == targets[n]] - p[n, v])
 *               + grad_entropy[n] * p[n, v] * (lse[n] - entropy[n] - z[n, v])
 *   out[n, v - vocab_begin] = bf16(dL/dz[n, v] / temperature)        (round to nearest even)
 * with lse and entropy as written by dsv41_logprob_run.  NULL grad_logprob or grad_entropy
 * counts as zero.  The logits are recomputed on the matrix cores, never stored in fp32.
 * dL/dx = out @ w[vocab_begin:vocab_end] and dL/dw[vocab_begin:vocab_end] = out^T @ x are
 * plain GEMMs left to the caller's BLAS.
 */
typedef struct dsv41_logprob_grad_desc {
  uint32_t struct_size; /* = sizeof(dsv41_logprob_grad_desc) */
  int32_t n_tokens;
  int32_t hidden;
  int32_t vocab;            /* rows of w */
  const void* x;            /* bf16 [N, H] */
  int64_t x_row_stride;     /* in elements, multiple of 8 */
  const void* w;            /* bf16 [V, H] */
  int64_t w_row_stride;     /* in elements, multiple of 8 */
  const int64_t* targets;   /* [N], each in [0, V) */
  float temperature;        /* finite, > 0; the forward's */
  const float* lse;         /* [N] */
  const float* entropy;     /* [N]; required when grad_entropy != NULL */
  const float* grad_logprob; /* [N] or NULL */
  const float* grad_entropy; /* [N] or NULL */
  int32_t vocab_begin;      /* 0 <= vocab_begin < vocab_end <= vocab */
  int32_t vocab_end;
  void* out;                /* bf16 [N, out_row_stride] */
  int64_t out_row_stride;   /* in elements, >= vocab_end - vocab_begin, multiple of 8 */
} dsv41_logprob_grad_desc;

/*
 * Decoupled Token-TIS loss over a packed batch of responses (response r owns tokens
 * [offsets[r], offsets[r+1]) of the per-token vectors; each response nonempty):
 *   delta = f32(native_old - behavior);  raw = exp(f64(delta));  w = f32(min(raw, is_cap))
 *   ratio = exp(f32(current - native_old))
 *   s = min(ratio * A_r, clamp(ratio, f32(1 - clip_eps), f32(1 + clip_eps)) * A_r)
 *   out_loss = mean_r( -mean_{i in r}(w_i * s_i) )                           (fp32)
 *   out_grad[i] = d out_loss / d current[i]  (torch's minimum / clamp gradient rules)
 *   out_metrics[DSV41_TIS_M_*]: the diagnostics of the reference's metric dict (fp64),
 *   pooled over all responses as aggregate_token_tis_metrics pools per-response rows.
 *   out_status[r]: DSV41_TIS_* bits of the reference's per-response checks.
 */
typedef struct dsv41_token_tis_desc {
  uint32_t struct_size; /* = sizeof(dsv41_token_tis_desc) */
  int32_t n_responses;  /* R > 0 */
  int64_t n_tokens;          /* length of the per-token vectors */
  const int64_t* offsets;    /* [R + 1], nondecreasing, in [0, n_tokens] */
  const float* current;      /* [tokens] learner log-probs */
  const float* native_old;   /* [tokens] */
  const float* behavior;     /* [tokens] */
  const float* advantages;   /* [R] */
  double clip_eps;           /* finite, in [0, 1) */
  double is_cap;             /* finite, > 0 */
  float* out_loss;           /* [1] or NULL */
  float* out_grad;           /* [tokens] or NULL */
  double* out_metrics;       /* [DSV41_TIS_METRICS] or NULL */
  int32_t* out_status;       /* [R] */
} dsv41_token_tis_desc;

/* out_status bits of dsv41_token_tis_run, in the reference's check order. */
#define DSV41_TIS_CURRENT_NONFINITE 0x1
#define DSV41_TIS_CURRENT_POSITIVE 0x2   /* a value > 1e-6 */
#define DSV41_TIS_OLD_NONFINITE 0x4
#define DSV41_TIS_OLD_POSITIVE 0x8
#define DSV41_TIS_BEHAVIOR_NONFINITE 0x10
#define DSV41_TIS_BEHAVIOR_POSITIVE 0x20
#define DSV41_TIS_RAW_NONFINITE 0x40
#define DSV41_TIS_RAW_ZERO 0x80
#define DSV41_TIS_WEIGHT_NONFINITE 0x100
#define DSV41_TIS_WEIGHT_ZERO 0x200
#define DSV41_TIS_RATIO_NONFINITE 0x400
#define DSV41_TIS_RATIO_ZERO 0x800
#define DSV41_TIS_EMPTY 0x1000
#define DSV41_TIS_ADV_NONFINITE 0x2000
#define DSV41_TIS_BAD_OFFSETS 0x4000     /* offsets outside [0, n_tokens] or decreasing */

/* out_metrics indices (the reference's metric keys, algorithm.py:322-346). */
#define DSV41_TIS_M_LOSS 0
#define DSV41_TIS_M_POLICY_LOSS 1
#define DSV41_TIS_M_RESPONSE_COUNT 2
#define DSV41_TIS_M_TOKEN_COUNT 3
#define DSV41_TIS_M_IS_CAP 4
#define DSV41_TIS_M_WEIGHT_SUM 5
#define DSV41_TIS_M_WEIGHT_SQUARE_SUM 6
#define DSV41_TIS_M_WEIGHT_MEAN 7
#define DSV41_TIS_M_WEIGHT_MIN 8
#define DSV41_TIS_M_WEIGHT_MAX 9
#define DSV41_TIS_M_RAW_WEIGHT_SUM 10
#define DSV41_TIS_M_RAW_WEIGHT_MIN 11
#define DSV41_TIS_M_RAW_WEIGHT_MAX 12
#define DSV41_TIS_M_CLIPPED_TOKENS 13
#define DSV41_TIS_M_CLIPPED_FRACTION 14
#define DSV41_TIS_M_DROPPED_MASS 15
#define DSV41_TIS_M_DROPPED_MASS_FRACTION 16
#define DSV41_TIS_M_ESS 17
#define DSV41_TIS_M_ESS_FRACTION 18
#define DSV41_TIS_M_DELTA_MEAN 19
#define DSV41_TIS_M_DELTA_MAX_ABS 20
#define DSV41_TIS_M_RATIO_MEAN 21
#define DSV41_TIS_M_RATIO_CLIP_FRACTION 22
#define DSV41_TIS_METRICS 23

/*
 * GRPO loss over a packed batch of responses (same packing as dsv41_token_tis_desc):
 *   ratio = exp(f32(current - behavior));  s = min(ratio A, clamp(ratio, f32(1-eps), f32(1+eps)) A)
 *   k3 = ratio * (expm1(reference - current) - (reference - current))   (kl_beta > 0)
 *   out_loss = mean_r(-mean_i s) + kl_beta * mean_r(mean_i k3)          (fp32)
 *   out_grad[i] = d out_loss / d current[i]
 *   out_metrics[DSV41_GRPO_M_*]: loss, policy_loss, kl, clip_fraction, importance_ratio,
 *   approx_kl as the reference's dict (means over responses of per-response means).
 */
typedef struct dsv41_grpo_desc {
  uint32_t struct_size; /* = sizeof(dsv41_grpo_desc) */
  int32_t n_responses;  /* R > 0 */
  int64_t n_tokens;
  const int64_t* offsets;   /* [R + 1], nondecreasing, in [0, n_tokens] */
  const float* current;     /* [tokens] */
  const float* behavior;    /* [tokens] */
  const float* reference;   /* [tokens]; required when kl_beta > 0 */
  const float* advantages;  /* [R] */
  double clip_eps;          /* finite, in [0, 1) */
  double kl_beta;           /* finite, >= 0 */
  float* out_loss;          /* [1] or NULL */
  float* out_grad;          /* [tokens] or NULL */
  double* out_metrics;      /* [DSV41_GRPO_METRICS] or NULL */
  int32_t* out_status;      /* [R] */
} dsv41_grpo_desc;

/* out_status bits of dsv41_grpo_run, in the reference's check order. */
#define DSV41_GRPO_CURRENT_NONFINITE 0x1
#define DSV41_GRPO_BEHAVIOR_NONFINITE 0x2
#define DSV41_GRPO_RATIO_NONFINITE 0x4
#define DSV41_GRPO_REFERENCE_NONFINITE 0x8
#define DSV41_GRPO_K3_NONFINITE 0x10
#define DSV41_GRPO_EMPTY 0x20
#define DSV41_GRPO_ADV_NONFINITE 0x40
#define DSV41_GRPO_BAD_OFFSETS 0x80

#define DSV41_GRPO_M_LOSS 0
#define DSV41_GRPO_M_POLICY_LOSS 1
#define DSV41_GRPO_M_KL 2
#define DSV41_GRPO_M_CLIP_FRACTION 3
#define DSV41_GRPO_M_IMPORTANCE_RATIO 4
#define DSV41_GRPO_M_APPROX_KL 5
#define DSV41_GRPO_METRICS 6

/* ABI identity. */
int dsv41_abi_version(void);
size_t dsv41_sampler_desc_size(void);
size_t dsv41_logprob_desc_size(void);
size_t dsv41_logprob_grad_desc_size(void);
size_t dsv41_token_tis_desc_size(void);
size_t dsv41_grpo_desc_size(void);
size_t dsv41_logprob_shard_desc_size(void);
size_t dsv41_logprob_combine_desc_size(void);
size_t dsv41_sampler_shard_desc_size(void);
size_t dsv41_sampler_merge_desc_size(void);
size_t dsv41_sampler_full_shard_desc_size(void);
size_t dsv41_sampler_full_finish_desc_size(void);
const char* dsv41_last_error(void);

/* Sampler: replaces rollout.py:144-150 for a [rows, vocab] batch.
 * Workspace (8-byte aligned, contents need no initialisation): rows*vocab*4 bytes for
 * top-p / min-p without top-k (the radix path); rows*(256*8+4) bytes for top-k batches
 * above 256 rows, whose rows hand up to 256 candidate keys and a count to a second
 * kernel on the same stream for the final selection; S*rows*(top_k*8+8) bytes for a
 * top-k batch (top_k <= 256) too small to fill the GPU, whose rows are split into S
 * 2048-aligned vocabulary slices of at least 6144 ids (up to about 256 workgroups in
 * all, S*top_k <= 4096) that
 * each leave their local top_k keys, a count and a status for a merge kernel on the
 * same stream; none otherwise. */
size_t dsv41_sampler_workspace_bytes(const dsv41_sampler_desc* desc);
int dsv41_sampler_run(const dsv41_sampler_desc* desc, void* workspace, size_t workspace_bytes,
                      void* stream /* hipStream_t */);

/* Sampler without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  It runs dsv41_sampler_run's kernels with the workspace taken
 * from a static device array of DSV41_SAMPLER_STATIC_SCRATCH_BYTES per GPU (held by every GPU
 * the library runs on until the process ends) and calls no allocator.  A batch whose
 * dsv41_sampler_workspace_bytes exceeds that size returns DSV41_E_UNSUPPORTED before any
 * launch (4096 rows of top-k need 8.4 MB; the radix path's rows*vocab*4 bytes fit only small
 * batches).  The stream must belong to the current device; the first call on a device looks
 * up the array's address there, so make it outside graph capture.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialised by the caller.  Nothing in the array needs clearing between
 * calls: each launch writes what it later reads. */
#define DSV41_SAMPLER_STATIC_SCRATCH_BYTES (32u << 20)
int dsv41_sampler_run_static(const dsv41_sampler_desc* desc, void* stream /* hipStream_t */);

/* Vocabulary-sharded sampler: per-slice candidate lists, then the exact merge (no workspace).
 * Together they replace rollout.py:144-150 when the head's vocabulary is split over GPUs;
 * the lists are what one all-gather would carry between the two calls. */
int dsv41_sampler_shard_run(const dsv41_sampler_shard_desc* desc, void* stream /* hipStream_t */);
int dsv41_sampler_merge_run(const dsv41_sampler_merge_desc* desc, void* stream /* hipStream_t */);

/* Vocabulary-sharded full-vocabulary draws: per-slice states, exact masses (inverse CDF
 * only), per-slice picks, then the finish (no workspace).  Together they replace
 * rollout.py:144-148 when the head's vocabulary is split over GPUs; states, masses and picks
 * are what the all-gathers carry. */
int dsv41_sampler_full_state_run(const dsv41_sampler_full_shard_desc* desc, void* stream /* hipStream_t */);
int dsv41_sampler_full_mass_run(const dsv41_sampler_full_shard_desc* desc, void* stream /* hipStream_t */);
int dsv41_sampler_full_draw_run(const dsv41_sampler_full_shard_desc* desc, void* stream /* hipStream_t */);
int dsv41_sampler_full_finish_run(const dsv41_sampler_full_finish_desc* desc, void* stream /* hipStream_t */);

/* Fused selected-token log-prob: replaces model.py:679-684 / native_lora.py:80-82. */
size_t dsv41_logprob_workspace_bytes(const dsv41_logprob_desc* desc);
int dsv41_logprob_run(const dsv41_logprob_desc* desc, void* workspace, size_t workspace_bytes,
                      void* stream /* hipStream_t */);

/* Vocabulary-sharded head: per-slice states, then the exact combine (no workspace). */
size_t dsv41_logprob_shard_workspace_bytes(const dsv41_logprob_shard_desc* desc);
int dsv41_logprob_shard_run(const dsv41_logprob_shard_desc* desc, void* workspace, size_t workspace_bytes,
                            void* stream /* hipStream_t */);
int dsv41_logprob_combine_run(const dsv41_logprob_combine_desc* desc, void* stream /* hipStream_t */);

/* Gradient of the fused log-prob with respect to the logits (no workspace). */
int dsv41_logprob_grad_run(const dsv41_logprob_grad_desc* desc, void* stream /* hipStream_t */);

/* Token-TIS loss, gradient and metrics: replaces algorithm.py:249-346 for a batch of
 * responses, pooled as distributed_grpo.py:197-222. */
size_t dsv41_token_tis_workspace_bytes(const dsv41_token_tis_desc* desc);
int dsv41_token_tis_run(const dsv41_token_tis_desc* desc, void* workspace, size_t workspace_bytes,
                        void* stream /* hipStream_t */);

/* GRPO loss, gradient and metrics: replaces algorithm.py:169-246 for a batch of responses. */
size_t dsv41_grpo_workspace_bytes(const dsv41_grpo_desc* desc);
int dsv41_grpo_run(const dsv41_grpo_desc* desc, void* workspace, size_t workspace_bytes,
                   void* stream /* hipStream_t */);

#ifdef __cplusplus
}
#endif

#endif /* DSV41_ROCM_H */
