/*
 * sampler_oracle.c — CPU restatement of the row-sampler specification.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker.  The product
 * (libdsv41hip.so) never links or calls it.
 *
 * What it restates (paths relative to the Tiny-DSV41 reference tree):
 *   - the sampling step of generate_group, dsv41_train/rl/rollout.py:144-150:
 *     z = logits.float() / T (IEEE division), log-prob of the drawn token under
 *     log_softmax(z), non-finite rows rejected (rollout.py:145-146);
 *   - greedy = first index of the maximum, dsv41_train/sft_eval.py:64 (argmax);
 *   - the vLLM SamplingParams knobs the rollout actor carries
 *     (rollout_manager/backends/vllm_actor.py:178-185, processed log-probs :260),
 *     in vLLM v1's order: penalties (repetition, frequency, presence), temperature,
 *     min-p, top-k, top-p.  vLLM itself is not installed; the spec below is the
 *     build's written definition of those knobs.
 *
 * Exactness: every decision that selects tokens is made in IEEE fp32 compares,
 * exact fp64 differences of fp32 values, and 64-bit fixed-point masses
 * (2^-43 resolution) whose sums are associative, so any reduction order gives the
 * same kept set and the same drawn id.  The only transcendental on that path is the
 * exponential inside dsv41_mass() below, a fixed sequence of fp32 operations; the
 * log-prob uses dsv41_exp_det(), a fixed sequence of fp64 operations.
 *
 * Every function here is pinned by tests/test_oracle_sampler.py against closed
 * forms (log_softmax in fp64, libm exp), brute force on tiny vocabularies, and
 * hand-derived penalty values.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ST_NONFINITE 1
#define ST_BAD_HISTORY 2
#define ST_BAD_UNIFORM 4

typedef unsigned __int128 u128;

/* ---- deterministic exp for d <= 0 (spec function) ------------------------- */
/* Cody-Waite reduction by ln2 split in two parts, degree-13 Taylor polynomial,
 * exact scaling by 2^n.  Returns 0 for d < -40 (e^-40 < 2^-57, below the 2^-43
 * mass resolution) and for NaN. */
double dsv41_exp_det(double d) {
  if (!(d >= -40.0)) return 0.0;
  if (d > 0.0) d = 0.0;
  const double log2e = 1.4426950408889634074;
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  double n = rint(d * log2e);
  double r = fma(-n, ln2_hi, d);
  r = fma(-n, ln2_lo, r);
  double p = 1.0 / 6227020800.0; /* 1/13! */
  p = fma(p, r, 1.0 / 479001600.0);
  p = fma(p, r, 1.0 / 39916800.0);
  p = fma(p, r, 1.0 / 3628800.0);
  p = fma(p, r, 1.0 / 362880.0);
  p = fma(p, r, 1.0 / 40320.0);
  p = fma(p, r, 1.0 / 5040.0);
  p = fma(p, r, 1.0 / 720.0);
  p = fma(p, r, 1.0 / 120.0);
  p = fma(p, r, 1.0 / 24.0);
  p = fma(p, r, 1.0 / 6.0);
  p = fma(p, r, 0.5);
  p = fma(p, r, 1.0);
  p = fma(p, r, 1.0);
  int64_t e = 1023 + (int64_t)n;
  uint64_t bits = (uint64_t)e << 52;
  double scale;
  memcpy(&scale, &bits, sizeof scale);
  return p * scale;
}

/* Fixed-point mass of a token: floor(2^43 * e) with e = exp(z - zmax) evaluated by a fixed
 * sequence of fp32 operations: d = z - zmax (fp32), 0 for d < -40 and NaN; Cody-Waite
 * reduction by a two-part ln 2, a degree-7 Taylor polynomial in Horner form with fma, and an
 * exact scale by 2^(n + 43).  Every step is an IEEE fp32 operation (fmaf, rintf, ldexpf,
 * floorf are exact or correctly rounded), so the device computes the same integer. */
uint64_t dsv41_mass(float z, float zmax) {
  float d = z - zmax;
  if (!(d >= -40.0f)) return 0;
  if (d > 0.0f) d = 0.0f;
  float n = rintf(d * 0x1.715476p+0f);   /* log2(e) */
  float r = fmaf(-n, 0x1.62e4p-1f, d);    /* ln 2, high part (exact products) */
  r = fmaf(-n, 0x1.7f7d1cp-20f, r);       /* ln 2, low part */
  float p = 0x1.a01a02p-13f;              /* 1/7! */
  p = fmaf(p, r, 0x1.6c16c2p-10f);        /* 1/6! */
  p = fmaf(p, r, 0x1.111112p-7f);         /* 1/5! */
  p = fmaf(p, r, 0x1.555556p-5f);         /* 1/4! */
  p = fmaf(p, r, 0x1.555556p-3f);         /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return (uint64_t)floorf(ldexpf(p, (int)n + 43));
}

/* ceil(p * s) exactly, p a positive fp32 <= 1. */
uint64_t dsv41_top_p_threshold(float p, uint64_t s) {
  uint32_t bits;
  memcpy(&bits, &p, sizeof bits);
  uint32_t be = (bits >> 23) & 0xFF;
  uint64_t mant = bits & 0x7FFFFF;
  int sh;
  if (be == 0) {
    sh = 149;
  } else {
    mant |= 0x800000;
    sh = 150 - (int)be; /* p = mant * 2^(be - 127 - 23) */
  }
  u128 prod = (u128)mant * s;
  if (prod == 0) return 0;
  if (sh <= 0) return (uint64_t)(prod << (-sh));
  if (sh >= 100) return 1;
  u128 one = (u128)1 << sh;
  return (uint64_t)((prod + one - 1) >> sh);
}

/* floor(u * 2^32) for a uniform in [0, 1); the draw target is (S * U) >> 32. */
uint64_t dsv41_draw_target(float u, uint64_t s) {
  uint64_t uu = (uint64_t)(u * 4294967296.0f);
  return (uint64_t)(((u128)s * uu) >> 32);
}

/* Penalties on one logit of an id in the history (vLLM v1 apply_penalties: repetition for
 * ids of the prompt or the output, then frequency * c and presence (c > 0), where c counts
 * the id among the generated entries only). */
float dsv41_penalize(float x, uint32_t c, float rp, float pres, float freq) {
  x = x > 0.0f ? x / rp : x * rp;
  float f = freq * (float)c;
  x = x - f;
  if (c > 0) x = x - pres;
  return x;
}

static inline uint32_t okey(float z) {
  uint32_t b;
  memcpy(&b, &z, sizeof b);
  if (b == 0x80000000u) b = 0; /* -0 ties with +0 */
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

static inline uint64_t ckey(float z, uint32_t idx) {
  return ((uint64_t)okey(z) << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

static int cmp_desc_u64(const void* a, const void* b) {
  uint64_t x = *(const uint64_t*)a, y = *(const uint64_t*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

static int cmp_asc_u32(const void* a, const void* b) {
  uint32_t x = *(const uint32_t*)a, y = *(const uint32_t*)b;
  return x < y ? -1 : (x > y ? 1 : 0);
}

/*
 * Processed logits of one row: z[v] for v < V.  The first plen history entries are the
 * prompt's (membership only), the rest the generated ids (counted).  counts[] is scratch of
 * V uint32: bit 31 marks membership, the low bits hold the generated count.
 * Returns status bits (NONFINITE / BAD_HISTORY).
 */
int dsv41_oracle_process_row(const float* x, int V, const int64_t* hist, int hlen, int plen, float T,
                             float rp, float pres, float freq, uint32_t* counts, float* z) {
  int status = 0;
  memset(counts, 0, sizeof(uint32_t) * (size_t)V);
  /* history is read only when a penalty is active: neutral knobs leave every logit as is
     and flag nothing */
  if (rp == 1.0f && pres == 0.0f && freq == 0.0f) hlen = 0;
  for (int j = 0; j < hlen; ++j) {
    int64_t id = hist[j];
    if (id < 0) continue;
    if (id >= V) {
      status |= ST_BAD_HISTORY;
      continue;
    }
    counts[id] |= 0x80000000u;
    if (j >= plen) counts[id] += 1;
  }
  for (int v = 0; v < V; ++v) {
    float xv = x[v];
    if (counts[v]) xv = dsv41_penalize(xv, counts[v] & 0x7FFFFFFFu, rp, pres, freq);
    float zv = xv / T;
    if (!isfinite(zv)) status |= ST_NONFINITE;
    z[v] = zv;
  }
  return status;
}

/*
 * Inverse-CDF draw over the whole row (no truncation) with 256-id chunk masses.  The row
 * is cut into chunks of MASS_CHUNK consecutive ids; chunks restart at every slice start
 * (starts[0..n_starts), ascending, starts[0] = 0; NULL = one slice).  An id outside the
 * history H (the ids the penalties processed, counts[v] != 0) weighs
 *   w_v = floor(2^43 exp32(z_v - m_c)),  m_c = max of z over the chunk's ids outside H,
 * and the chunk weighs Q_c = floor(W_c g_c / 2^43) + sum over its ids in H of
 * floor(2^43 exp32(z_h - zmax)), with W_c = sum w_v and g_c = floor(2^43 exp32(m_c - zmax)).
 * The target t = (S U) >> 32 with S = sum Q_c picks the first chunk whose cumulative Q
 * exceeds t; inside it, the id boundaries in Q units are floor(prefix(w) g_c / 2^43) +
 * prefix(history masses), in vocabulary order, and the first boundary above what the chunk
 * owes names the token.  Every quantity is an integer, so sums in any order agree.
 */
#define MASS_CHUNK 256
/* The chunk [lo, hi)'s maximum over ids outside H (mc), its g and its weight Q. */
static uint64_t chunk_weight(const float* z, int lo, int hi, const uint32_t* counts, float zmax, float* mc_out,
                             uint64_t* g_out) {
  float mc = -INFINITY;
  for (int v = lo; v < hi; ++v)
    if (!(counts && counts[v]) && z[v] > mc) mc = z[v];
  const uint64_t g = dsv41_mass(mc, zmax);
  uint64_t W = 0, Hm = 0;
  for (int v = lo; v < hi; ++v) {
    if (counts && counts[v]) Hm += dsv41_mass(z[v], zmax);
    else W += dsv41_mass(z[v], mc);
  }
  *mc_out = mc;
  *g_out = g;
  return (uint64_t)(((u128)W * g) >> 43) + Hm;
}

/* S = sum Q_c over the chunks of every slice: the total every full-vocabulary draw reports
 * its log-prob against, lp = (z_tok - zmax) - log(S 2^-43). */
static uint64_t full_total(const float* z, int V, const uint32_t* counts, const int32_t* starts, int n_starts,
                           float zmax) {
  uint64_t S = 0;
  for (int s = 0; s < (starts ? n_starts : 1); ++s) {
    const int a = starts ? starts[s] : 0;
    const int b = (starts && s + 1 < n_starts) ? starts[s + 1] : V;
    for (int lo = a; lo < b; lo += MASS_CHUNK) {
      float mc;
      uint64_t g;
      S += chunk_weight(z, lo, lo + MASS_CHUNK < b ? lo + MASS_CHUNK : b, counts, zmax, &mc, &g);
    }
  }
  return S;
}

static int64_t full_draw(const float* z, int V, const uint32_t* counts, const int32_t* starts, int n_starts,
                         float zmax, uint64_t U) {
  const uint64_t S = full_total(z, V, counts, starts, n_starts, zmax);
  const uint64_t t = (uint64_t)(((u128)S * U) >> 32); /* dsv41_draw_target with U = u 2^32 */
  uint64_t before = 0;
  for (int s = 0; s < (starts ? n_starts : 1); ++s) {
    const int a = starts ? starts[s] : 0;
    const int b = (starts && s + 1 < n_starts) ? starts[s + 1] : V;
    for (int lo = a; lo < b; lo += MASS_CHUNK) {
      const int hi = lo + MASS_CHUNK < b ? lo + MASS_CHUNK : b;
      float mc;
      uint64_t g;
      const uint64_t Q = chunk_weight(z, lo, hi, counts, zmax, &mc, &g);
      if (t < before + Q) {
        const uint64_t need = t - before;
        uint64_t cw = 0, ch = 0;
        for (int v = lo; v < hi; ++v) {
          if (counts && counts[v]) ch += dsv41_mass(z[v], zmax);
          else cw += dsv41_mass(z[v], mc);
          if (need < (uint64_t)(((u128)cw * g) >> 43) + ch) return v;
        }
      }
      before += Q;
    }
  }
  return -1; /* no mass: only rows without a finite maximum */
}

/* The exact total S of processed logits z[V] (maximum taken over z). */
uint64_t dsv41_oracle_full_total(const float* z, int V, const uint32_t* counts, const int32_t* starts,
                                 int n_starts) {
  float zmax = z[0];
  for (int v = 1; v < V; ++v)
    if (z[v] > zmax) zmax = z[v];
  return full_total(z, V, counts, starts, n_starts, zmax);
}

/* The full-vocabulary inverse-CDF draw of processed logits z[V] against the 32-bit
 * uniform U (the draw of u = U / 2^32), for the tests' interval checks. */
int64_t dsv41_oracle_full_draw(const float* z, int V, const uint32_t* counts, const int32_t* starts,
                               int n_starts, uint32_t U) {
  float zmax = z[0];
  for (int v = 1; v < V; ++v)
    if (z[v] > zmax) zmax = z[v];
  return full_draw(z, V, counts, starts, n_starts, zmax, U);
}

/*
 * Kept set + draw for one row of processed logits z[V].
 * Writes *id, *lp, *kept; returns status bits (BAD_UNIFORM).
 * scratch_keys: V uint64, scratch_idx: V uint32.  counts: the history membership of
 * dsv41_oracle_process_row (NULL: none); starts / n_starts: slice starts of the
 * full-vocabulary draw's chunks (NULL: one slice).
 */
int dsv41_oracle_select_row(const float* z, int V, float u, int top_k, float top_p, float min_p,
                            int greedy, uint64_t* keys, uint32_t* idxs, int64_t* out_id,
                            float* out_lp, int32_t* out_kept, const uint32_t* counts,
                            const int32_t* starts, int n_starts) {
  int status = 0;
  /* first index of the maximum */
  int am = 0;
  float zmax = z[0];
  for (int v = 1; v < V; ++v)
    if (z[v] > zmax) {
      zmax = z[v];
      am = v;
    }
  const int truncating = (min_p > 0.0f) || (top_k > 0 && top_k < V) || (top_p < 1.0f);
  int n_keep;
  if (!truncating) {
    n_keep = V;
    for (int v = 0; v < V; ++v) idxs[v] = (uint32_t)v;
  } else {
    double lmin = min_p > 0.0f ? log((double)min_p) : -INFINITY;
    int n = 0;
    for (int v = 0; v < V; ++v) {
      if (min_p > 0.0f && !((double)z[v] - (double)zmax >= lmin)) continue;
      keys[n++] = ckey(z[v], (uint32_t)v);
    }
    qsort(keys, (size_t)n, sizeof(uint64_t), cmp_desc_u64);
    int kk = (top_k > 0 && top_k < n) ? top_k : n;
    n_keep = kk;
    if (top_p < 1.0f) {
      uint64_t s = 0;
      for (int i = 0; i < kk; ++i) {
        uint32_t v = 0xFFFFFFFFu - (uint32_t)(keys[i] & 0xFFFFFFFFu);
        s += dsv41_mass(z[v], zmax);
      }
      uint64_t thr = dsv41_top_p_threshold(top_p, s);
      uint64_t c = 0;
      for (int i = 0; i < kk; ++i) {
        uint32_t v = 0xFFFFFFFFu - (uint32_t)(keys[i] & 0xFFFFFFFFu);
        c += dsv41_mass(z[v], zmax);
        if (c >= thr) {
          n_keep = i + 1;
          break;
        }
      }
    }
    for (int i = 0; i < n_keep; ++i) idxs[i] = 0xFFFFFFFFu - (uint32_t)(keys[i] & 0xFFFFFFFFu);
    qsort(idxs, (size_t)n_keep, sizeof(uint32_t), cmp_asc_u32);
  }
  /* kept set in vocabulary order: idxs[0..n_keep) */
  uint64_t s = 0;
  double esum = 0.0;
  for (int i = 0; i < n_keep; ++i) {
    uint32_t v = idxs[i];
    s += dsv41_mass(z[v], zmax);
    esum += dsv41_exp_det((double)z[v] - (double)zmax);
  }
  int64_t tok;
  if (greedy) {
    tok = am;
  } else if (!truncating) {
    float uu = u;
    if (!(uu >= 0.0f && uu < 1.0f)) {
      status |= ST_BAD_UNIFORM;
      uu = 0.0f;
    }
    tok = full_draw(z, V, counts, starts, n_starts, zmax, (uint64_t)(uu * 4294967296.0f));
    if (tok < 0) tok = am;
  } else {
    float uu = u;
    if (!(uu >= 0.0f && uu < 1.0f)) {
      status |= ST_BAD_UNIFORM;
      uu = 0.0f;
    }
    uint64_t t = dsv41_draw_target(uu, s);
    uint64_t c = 0;
    tok = idxs[n_keep - 1];
    for (int i = 0; i < n_keep; ++i) {
      c += dsv41_mass(z[idxs[i]], zmax);
      if (c > t) {
        tok = idxs[i];
        break;
      }
    }
  }
  *out_id = tok;
  *out_lp = (float)(((double)z[tok] - (double)zmax) - log(esum));
  *out_kept = n_keep;
  return status;
}

/*
 * Whole batch.  logits fp32 [rows, V] (bf16 inputs are widened exactly by the
 * caller), history int64 [rows, hstride] with per-row lengths (or hlen).
 * Non-finite rows get id -1, NaN log-prob and kept 0.
 */
int dsv41_oracle_sample(const float* logits, int rows, int V, const int64_t* hist,
                        int64_t hstride, int hlen, const int32_t* hlens, const int32_t* plens,
                        const float* uniforms,
                        float T, float rp, float pres, float freq, int top_k, float top_p,
                        float min_p, int greedy, int64_t* out_ids, float* out_lp,
                        int32_t* out_kept, int32_t* out_status, const int32_t* slice_starts,
                        int n_slices) {
  uint32_t* counts = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)V);
  float* z = (float*)malloc(sizeof(float) * (size_t)V);
  uint64_t* keys = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)V);
  uint32_t* idxs = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)V);
  if (!counts || !z || !keys || !idxs) {
    free(counts);
    free(z);
    free(keys);
    free(idxs);
    return -1;
  }
  for (int r = 0; r < rows; ++r) {
    int hl = hist ? (hlens ? hlens[r] : hlen) : 0;
    int st = dsv41_oracle_process_row(logits + (size_t)r * V, V, hist ? hist + r * hstride : NULL,
                                      hl, plens ? plens[r] : 0, T, rp, pres, freq, counts, z);
    if (st & ST_NONFINITE) {
      out_ids[r] = -1;
      out_lp[r] = NAN;
      out_kept[r] = 0;
      out_status[r] = st;
      continue;
    }
    float u = uniforms ? uniforms[r] : 0.0f;
    st |= dsv41_oracle_select_row(z, V, u, top_k, top_p, min_p, greedy, keys, idxs, &out_ids[r],
                                  &out_lp[r], &out_kept[r], counts, slice_starts, n_slices);
    out_status[r] = st;
  }
  free(counts);
  free(z);
  free(keys);
  free(idxs);
  return 0;
}

/*
 * Checks the kernel's three-operation division scheme against IEEE division on
 * every fp32 bit pattern x with lo <= (bits of x) < hi:
 *   r = RN(1/T); q = RN(x*r); e = fma(-q, T, x); z = fma(e, r, q)   ==?   x / T
 * (Markstein's correction step).  Non-finite quotients are skipped: such rows are
 * reported non-finite either way.  Returns the number of mismatches; *first gets
 * the first mismatching bit pattern.
 */
uint64_t dsv41_check_division(float T, uint32_t lo, uint32_t hi, uint32_t* first) {
  float r = 1.0f / T;
  uint64_t bad = 0;
  for (uint64_t b = lo; b < hi; ++b) {
    uint32_t bb = (uint32_t)b;
    float x;
    memcpy(&x, &bb, sizeof x);
    float ref = x / T;
    if (!isfinite(ref) || !isfinite(x)) continue;
    float q = x * r;
    float e = fmaf(-q, T, x);
    float zz = fmaf(e, r, q);
    uint32_t a, c;
    memcpy(&a, &ref, 4);
    memcpy(&c, &zz, 4);
    if (a != c) {
      if (!bad && first) *first = bb;
      ++bad;
    }
  }
  return bad;
}
