// sampler.hip — row sampler for gfx950: penalties over per-row history, temperature,
// min-p / top-k / top-p, greedy or inverse-CDF draw against caller uniforms, and the
// drawn token's log-prob under the processed distribution.
//
// Replaces the sampling step of generate_group (dsv41_train/rl/rollout.py:144-150:
// log_softmax(logits.float() / T), finite check, draw, behaviour log-prob) for a
// [rows, vocab] batch, with the vLLM SamplingParams knobs of
// rollout_manager/backends/vllm_actor.py:178-185 applied in vLLM v1's order.
//
// One workgroup per row streams the row from HBM exactly once, through raw buffer
// loads (out-of-range lanes read 0, so the pipeline has no branches around loads),
// double-buffered in batches of PF tiles:
//   FULL    (no truncation): per-chunk (max, sum exp) in LDS for the row maximum and the
//           log-prob's total; an inverse-CDF draw streams the row once more for each
//           chunk's exact fixed-point mass, then re-reads one 64*G-element chunk to place
//           the token.
//   TOPK    (1 <= top_k <= 2048): elements above a running threshold (top-k of what
//           has been seen, and the min-p bound of the running maximum) go to an LDS
//           candidate buffer; after the pass the buffer is sorted and every decision
//           (min-p, top-k, top-p, draw) is an exact scan over it.
//   TOPP    (top-p alone): three streams of the row.  The first finds the maximum; the
//           second sums every token's exact mass into the row total and into bins of
//           the float bits of (max - z); the third collects the bin holding the top-p
//           boundary and the kept mass of every 64*G-element chunk for the draw.
//   GENERIC (anything else that truncates): z is written to a workspace row and the
//           same decisions are made by exact radix selection over it.
// History tokens are masked out of the stream and re-read per batch from the lines
// the batch has just brought on chip, then penalized exactly.
// Selection arithmetic is exact (fp32 compares, fp64 differences of fp32 values,
// 64-bit fixed-point masses), so kept sets and ids do not depend on reduction order.
// This file is compiled with -ffp-contract=off: each operation rounds as written.

#include <math.h>
#include <limits.h>
#include <string.h>

#include <mutex>
#include <string>
#include <type_traits>

#include "common.h"

namespace dsv41 {
namespace sampler {

constexpr int MODE_FULL = 0;
constexpr int MODE_TOPK = 1;
constexpr int MODE_GENERIC = 2;
constexpr int MODE_TOPP = 3;

constexpr int FULL_NT = 1024;
constexpr int TOPK_NT = 512;
constexpr int GEN_NT = 1024;
constexpr int FALLBACK_GRID = 512;             // generic_kernel workgroups of a fallback launch
constexpr int MAX_NW = 16;
constexpr int PF = 4;                          // tiles per pipelined batch
constexpr int TOPK_G = 4;                      // elements per thread per TOPK tile
constexpr int TOPK_TILE = TOPK_NT * TOPK_G;    // 2048
constexpr int KCAP = TOPK_TILE;                // largest top_k on the one-pass path
constexpr int MAX_VOCAB = (1 << 21) - 1;       // (2^21 - 1) masses of at most 2^43 sum below 2^64
constexpr int MAX_UNIQUE = 65535;              // history slots and counts are 16-bit
constexpr int DEFER_KEYS = 4 * 64;             // candidates a one-wave final selection holds
constexpr int DEFER_MIN_ROWS = 256;            // batches above one row per CU defer it
constexpr int SEL_WAVES = 4;                   // rows per select_kernel workgroup
constexpr int INTERNAL_K = 1024;               // min-p without top-k: the bound topk_kernel keeps
                                               // (its buffer then leaves room for two workgroups per CU)
constexpr int TOPP_NT = 1024;
constexpr int TOPP_BINS = 4096;                // 32 octaves of (max - z) x 128 steps
constexpr int TOPP_BIN_BASE = 100 << 7;        // octave 0 is [2^-27, 2^-26); smaller -> bin 0
constexpr int TOPP_CAP = 4096;                 // list / boundary-bin tokens topp_kernel holds
static_assert(TOPP_CAP <= TOPP_BINS, "the boundary bin's tokens from the list go to the bins' space");
constexpr size_t LDS_LIMIT = 160 * 1024;
// Cache policy of the row streams: nt (non-temporal).  A pass reads each logit and history
// id once, so its lines should not take L2 or Infinity Cache space from data that is
// reused.  At E (4096 x 151936 fp32) this took a launch from 483 to 437 us, and top-p
// (three reads of a row) is unchanged.
constexpr int STREAM_CPOL = 2;
constexpr int FULL_CPOL = 0;  // full_kernel's exact draw re-reads each row: default caching

constexpr float NEG_INF = -__builtin_huge_valf();
constexpr uint32_t NEG_INF_BITS = 0xFF800000u;

constexpr int ST_NONFINITE = DSV41_STATUS_NONFINITE;
constexpr int ST_BAD_HISTORY = DSV41_STATUS_BAD_HISTORY;
constexpr int ST_BAD_UNIFORM = DSV41_STATUS_BAD_UNIFORM;
constexpr int ST_BAD_TARGET = DSV41_STATUS_BAD_TARGET;
constexpr int ST_BAD_SLICES = DSV41_STATUS_BAD_SLICES;
constexpr int ST_RECHECK = 1 << 30;  // internal to topk_kernel: re-check every element of the row
constexpr int ST_FALLBACK = 1 << 29; // internal: an internal-k TOPK row needs generic_kernel

// full_kernel draws
constexpr int DRAW_CDF = 0;     // inverse CDF against one uniform
constexpr int DRAW_RACE = 1;    // exponential race against Exp(1) variates
constexpr int DRAW_REPLAY = 2;  // no draw: the log-prob of a given token
// vocabulary slices of a full-vocabulary draw (dsv41_sampler_full_*_run)
constexpr int DRAW_STATE = 3;       // the slice's state: max, exact mass total, first argmax
constexpr int DRAW_SHARD_CDF = 4;   // inverse CDF against the gathered states
constexpr int DRAW_SHARD_RACE = 5;  // exponential race against the gathered states
constexpr int DRAW_SHARD_MASS = 6;  // the slice's exact fixed-point mass against the gathered maximum
constexpr int DRAW_GREEDY = 7;      // first largest logit, no draw
constexpr int DRAW_ARGMAX = 8;      // first largest logit without its log-prob: no masses
// Exact masses of the inverse-CDF draws are formed per chunk of MASS_CHUNK consecutive ids
// of the row (or slice), against the chunk's own maximum.
constexpr int MASS_CHUNK = 256;
// FULL batches of at most this many rows are spread over the GPU
constexpr int PRE_MAX_ROWS = 128;
constexpr size_t PRE_MAX_LDS = 48 * 1024;  // a spread slice's history bitmap

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

struct Params {
  const void* logits;
  int64_t lstride;
  const int64_t* hist;
  int64_t hstride;
  const int32_t* hlens;
  const int32_t* plens;  // [rows] or NULL: leading history entries of the prompt (not counted)
  const float* uniforms;
  int64_t* out_ids;
  float* out_lp;
  int32_t* out_kept;
  int32_t* out_status;
  float* zbuf;
  const float* exps;  // exponential-race draw: [rows, estride] Exp(1) variates, or NULL
  int64_t estride;
  const int64_t* replay;  // DRAW_REPLAY: the token of each row
  double log_min_p;
  float T, rT, rp, pres, freq, top_p, min_p, lmin_f;
  int V, hlen, top_k, greedy, has_pen, unit_T, fast_div, ucap, words, cap;
  int pen_lowers;  // penalties can only lower a logit: rp >= 1, presence >= 0, frequency >= 0
  int pen_counts;  // the penalty of a history id depends on its count (frequency, or presence
                   // with prompt ids that count zero)
  // TOPK rows whose candidates fit one wave leave them here for select_kernel:
  // defer_keys[row * DEFER_KEYS + i], defer_count[row] (0: the row was finished in place)
  uint64_t* defer_keys;
  int32_t* defer_count;
  int defer;
  // vocabulary shard (topk_kernel<..., EMIT>): this launch sees ids [voff, voff + V) of a
  // vocab_size = vfull vocabulary and emits each row's candidates instead of sampling
  int voff, vfull, emit_cap;
  uint64_t* emit_keys;  // [rows, emit_cap]
  int32_t* emit_count;  // [rows]
  // min-p without top-k on topk_kernel: top_k holds an internal bound; a row that would
  // cut its min-p survivors at it is flagged ST_FALLBACK and redone by generic_kernel,
  // which then runs only on flagged rows (only_flagged)
  int topk_internal, only_flagged;
  // TOPK buffer size above which a batch compacts mid-stream (2 top_k + 128); none under
  // the internal bound, where a compaction against the running maximum could cut min-p
  // survivors that the final bound keeps
  int mid_trigger;
  // full-vocabulary draw over slices (DRAW_STATE / DRAW_SHARD_*): states [n_shards, nrows]
  const dsv41_full_state* sh_states;
  dsv41_full_state* sh_out_states;
  dsv41_full_pick* sh_out_picks;
  const uint64_t* sh_masses;  // [n_shards, nrows] gathered exact masses (DRAW_SHARD_CDF)
  uint64_t* sh_out_masses;    // [nrows] (DRAW_SHARD_MASS)
  int n_shards, shard_index, nrows;  // nrows: the batch's rows (also generic_kernel's fallback launch)
  // sliced small batch (topk_kernel<..., EMIT, NTK, SLICED>): workgroup b takes slice
  // b % n_slices (slice_w ids from slice * slice_w) of row b / n_slices
  int n_slices, slice_w;
  // TOPK with lowering penalties and no frequency penalty needs only the membership
  // bitmap: ucap is 0 then and the rank table is left out of the layout
  int no_ranks;
  // small FULL batch spread over the GPU: full_slice_kernel writes each row's wave-span
  // sums [rows, NC], 256-id chunk maxima and exact masses [rows, NE] and per-slice status
  // [rows, n_slices] (slice_w wave spans per slice); full_kernel<..., PRE> finishes rows
  float* pre_em;
  uint64_t* pre_w;
  int32_t* pre_st;
};

// Per-workgroup scalars and reduction scratch, at the start of dynamic LDS.
struct Misc {
  double rd[MAX_NW];
  uint64_t ru[MAX_NW];
  float rf[MAX_NW];
  float wmax[2][MAX_NW];
  int ri[MAX_NW];
  int wcnt[2][MAX_NW];
  uint64_t bu[4];
  double bd[4];
  float bf[4];
  int bi[4];
  int status;
  int count;
  int U;
  float tau;
  uint64_t tau_key;
  int unsorted;  // merge_kernel: some list is not in descending order
};

struct Layout {
  size_t misc, bitmap, wrank, cnt, tok, penx, hist256, mode0, total;
};

__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

template <int G>
__host__ __device__ inline int n_chunks(int V) {
  return (V + 64 * G - 1) / (64 * G);
}
__host__ __device__ inline int n_mass_chunks(int V) { return (V + MASS_CHUNK - 1) / MASS_CHUNK; }

// LDS layout; must agree between the launch (host) and the kernel (device).
// bitmap u32[words] | wrank u16[words] | cnt u16[ucap] | tok u32[ucap] |
// penx f32[ucap] (FULL) | 256 u64 radix bins | chunks (FULL: u64 exact mass[NE], f32
// max[NE], f32 sum[NC]; NE 256-id mass chunks, NC wave spans of one or two of them) or
// candidates (TOPK)
// ranks = false: the membership bitmap alone (no rank, count or token tables).
template <int MODE, int G>
__host__ __device__ inline Layout make_layout(int V, int words, int ucap, int cap, bool ranks = true) {
  Layout l;
  size_t off = 0;
  l.misc = off;
  off = align16(off + sizeof(Misc));
  l.bitmap = off;
  off += 4 * (size_t)words;
  l.wrank = off;
  off = align16(off + 2 * (size_t)(ranks ? words : 0));
  l.cnt = off;
  off = align16(off + 2 * (size_t)((ucap + 1) & ~1));
  l.tok = off;
  off = align16(off + 4 * (size_t)ucap);
  l.penx = off;
  if (MODE == MODE_FULL) off = align16(off + 4 * (size_t)ucap);
  l.hist256 = off;
  off += 256 * 8;
  l.mode0 = off;
  if (MODE == MODE_FULL) off += 12 * (size_t)n_mass_chunks(V);
  if (MODE == MODE_TOPK) off += 8 * (size_t)cap;
  if (MODE == MODE_TOPP) off += 8 * ((size_t)TOPP_BINS + (size_t)n_chunks<G>(V) + (size_t)cap);
  l.total = align16(off);
  return l;
}

// ------------------------------------------------------------ exact helpers
// Same specification as the oracle: Cody-Waite reduction, degree-13 Taylor
// polynomial in Horner form with fma, exact 2^n scaling; 0 below -40.
__device__ __forceinline__ double exp_det(double d) {
  if (!(d >= -40.0)) return 0.0;
  if (d > 0.0) d = 0.0;
  const double log2e = 1.4426950408889634074;
  const double ln2_hi = 6.93147180369123816490e-01;
  const double ln2_lo = 1.90821492927058770002e-10;
  double n = __builtin_rint(d * log2e);
  double r = __builtin_fma(-n, ln2_hi, d);
  r = __builtin_fma(-n, ln2_lo, r);
  double p = 1.0 / 6227020800.0;
  p = __builtin_fma(p, r, 1.0 / 479001600.0);
  p = __builtin_fma(p, r, 1.0 / 39916800.0);
  p = __builtin_fma(p, r, 1.0 / 3628800.0);
  p = __builtin_fma(p, r, 1.0 / 362880.0);
  p = __builtin_fma(p, r, 1.0 / 40320.0);
  p = __builtin_fma(p, r, 1.0 / 5040.0);
  p = __builtin_fma(p, r, 1.0 / 720.0);
  p = __builtin_fma(p, r, 1.0 / 120.0);
  p = __builtin_fma(p, r, 1.0 / 24.0);
  p = __builtin_fma(p, r, 1.0 / 6.0);
  p = __builtin_fma(p, r, 0.5);
  p = __builtin_fma(p, r, 1.0);
  p = __builtin_fma(p, r, 1.0);
  long long e = 1023 + (long long)n;
  return p * __longlong_as_double(e << 52);
}

// Fixed-point mass of a token, floor(2^43 * exp(z - zmax)), as an exact integer-valued
// float: the same fp32 operations as the oracle's specification (d = z - zmax, 0 below -40
// and for NaN; Cody-Waite reduction by a two-part ln 2; degree-7 Taylor polynomial in
// Horner form with fma; exact scale by 2^(n + 43); floor).  The range checks are one clamp
// here: fmaxf takes -40 for NaN, and d = -40 itself yields floor(2^43 e^-40 (1 + eps)) = 0,
// so every d the oracle maps to 0 gives 0.  Every step is exact or correctly rounded, so
// the integer is the oracle's bit for bit.  The result has at most 24 significant bits and
// is at most 2^43.
__device__ __forceinline__ float mass_ff(float z, float zmax) {
  float d = z - zmax;
  d = fminf(fmaxf(d, -40.0f), 0.0f);
  const float n = __builtin_rintf(d * 0x1.715476p+0f);
  float r = __builtin_fmaf(-n, 0x1.62e4p-1f, d);
  r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
  // The coefficients carry the 2^43: every Horner value is 2^43 times the unscaled one,
  // rounding included (all values stay normal), so only the 2^n scale remains.
  float p = 0x1.a01a02p+30f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p+33f);
  p = __builtin_fmaf(p, r, 0x1.111112p+36f);
  p = __builtin_fmaf(p, r, 0x1.555556p+38f);
  p = __builtin_fmaf(p, r, 0x1.555556p+40f);
  p = __builtin_fmaf(p, r, 0x1p+42f);
  p = __builtin_fmaf(p, r, 0x1p+43f);
  p = __builtin_fmaf(p, r, 0x1p+43f);
  return __builtin_floorf(__builtin_ldexpf(p, (int)n));
}

__device__ __forceinline__ uint64_t mass_of(float z, float zmax) { return (uint64_t)mass_ff(z, zmax); }

__device__ __forceinline__ uint64_t top_p_threshold(float p, uint64_t s) {
  uint32_t bits = __float_as_uint(p);
  uint32_t be = (bits >> 23) & 0xFF;
  uint64_t mant = bits & 0x7FFFFF;
  int sh;
  if (be == 0) {
    sh = 149;
  } else {
    mant |= 0x800000;
    sh = 150 - (int)be;
  }
  unsigned __int128 prod = (unsigned __int128)mant * s;
  if (prod == 0) return 0;
  if (sh <= 0) return (uint64_t)(prod << (-sh));
  if (sh >= 100) return 1;
  unsigned __int128 one = (unsigned __int128)1 << sh;
  return (uint64_t)((prod + one - 1) >> sh);
}

__device__ __forceinline__ uint64_t draw_target(float u, uint64_t s) {
  uint64_t uu = (uint64_t)(u * 4294967296.0f);
  return (uint64_t)(((unsigned __int128)s * uu) >> 32);
}

__device__ __forceinline__ float penalize(float x, uint32_t c, const Params& p) {
  x = x > 0.0f ? x / p.rp : x * p.rp;
  float f = p.freq * (float)c;
  x = x - f;
  if (c > 0) x = x - p.pres;  // c = 0: an id of the prompt only (repetition alone)
  return x;
}

__device__ __forceinline__ uint32_t okey(float z) {
  uint32_t b = __float_as_uint(z);
  if (b == 0x80000000u) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
// (z desc, index asc) order as a descending u64 order; unique per element.
__device__ __forceinline__ uint64_t ckey(float z, uint32_t idx) {
  return ((uint64_t)okey(z) << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}
__device__ __forceinline__ float ckey_z(uint64_t k) { return okey_inv((uint32_t)(k >> 32)); }
__device__ __forceinline__ uint32_t ckey_idx(uint64_t k) {
  return 0xFFFFFFFFu - (uint32_t)(k & 0xFFFFFFFFu);
}

__device__ __forceinline__ bool minp_ok(float z, float zmax, const Params& p) {
  return !(p.min_p > 0.0f) || ((double)z - (double)zmax >= p.log_min_p);
}

// ------------------------------------------------------------ block reductions
template <int NT>
__device__ __forceinline__ float block_max(float v, Misc* m) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_max_dpp(v);
  if (lane == 0) m->rf[wid] = v;
  __syncthreads();
  float r = m->rf[0];
  for (int i = 1; i < NW; ++i) r = fmaxf(r, m->rf[i]);
  __syncthreads();
  return r;
}
template <int NT>
__device__ __forceinline__ int block_sum_i(int v, Misc* m) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum_i(v);
  if (lane == 0) m->ri[wid] = v;
  __syncthreads();
  int r = 0;
  for (int i = 0; i < NW; ++i) r += m->ri[i];
  __syncthreads();
  return r;
}
template <int NT>
__device__ __forceinline__ int block_min_i(int v, Misc* m) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_min_i(v);
  if (lane == 0) m->ri[wid] = v;
  __syncthreads();
  int r = m->ri[0];
  for (int i = 1; i < NW; ++i) r = min(r, m->ri[i]);
  __syncthreads();
  return r;
}
template <int NT>
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, Misc* m) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum_u64(v);
  if (lane == 0) m->ru[wid] = v;
  __syncthreads();
  uint64_t r = 0;
  for (int i = 0; i < NW; ++i) r += m->ru[i];
  __syncthreads();
  return r;
}
template <int NT>
__device__ __forceinline__ double block_sum_d(double v, Misc* m) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum_d(v);
  if (lane == 0) m->rd[wid] = v;
  __syncthreads();
  double r = 0.0;
  for (int i = 0; i < NW; ++i) r += m->rd[i];
  __syncthreads();
  return r;
}

// In-place inclusive prefix sum of a[0..n).
template <int NT>
__device__ __forceinline__ void block_incl_scan_u64(uint64_t* a, int n, Misc* m) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int per = (n + NT - 1) / NT;
  const int b = tid * per, e = min(b + per, n);
  uint64_t s = 0;
  for (int i = b; i < e; ++i) s += a[i];
  uint64_t incl = wave_incl_scan_u64(s, lane);
  if (lane == 63) m->ru[wid] = incl;
  __syncthreads();
  uint64_t off = 0;
  for (int i = 0; i < wid; ++i) off += m->ru[i];
  uint64_t run = off + incl - s;
  for (int i = b; i < e; ++i) {
    run += a[i];
    a[i] = run;
  }
  __syncthreads();
}

// Descending sort of a[0..n) (u64 keys) by the bitonic network in its one-direction
// form (each merge starts with a mirror step, then half-cleaners; every comparator
// puts the larger key at the lower index).  Positions >= n act as keys below every
// real key and are never touched, so n need not be a power of two.
template <int NT>
__device__ __forceinline__ void bitonic_sort_desc(uint64_t* a, int n) {
  const int tid = threadIdx.x;
  int P = 1;
  while (P < n) P <<= 1;
  for (int k = 2; k <= P; k <<= 1) {
    // mirror step inside each k-block
    for (int i = tid; i < (P >> 1); i += NT) {
      const int half = k >> 1;
      const int blk = i / half, off = i - blk * half;
      const int lo = blk * k + off, hi = blk * k + (k - 1 - off);
      if (hi < n) {
        const uint64_t x = a[lo], y = a[hi];
        if (x < y) {
          a[lo] = y;
          a[hi] = x;
        }
      }
    }
    __syncthreads();
    for (int j = k >> 2; j > 0; j >>= 1) {
      for (int i = tid; i < (P >> 1); i += NT) {
        const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int hi = lo + j;
        if (hi < n) {
          const uint64_t x = a[lo], y = a[hi];
          if (x < y) {
            a[lo] = y;
            a[hi] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Radix selection.  Among elements offered by `visit(f)` (which calls f(key, weight)
// for each of this thread's elements), finds the key of the element at which the
// cumulative weight, taken in descending (DESC) or ascending key order, first reaches
// `target` (>= 1).  Keys must be unique; weight-0 elements are never chosen.  Returns
// the key, or 0 with *found = false when the total weight is below target.
template <int NT, bool DESC, int NBITS, class Visit>
__device__ __forceinline__ uint64_t radix_select(Visit visit, uint64_t target, uint64_t* hist, Misc* m,
                                 bool* found) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  uint64_t prefix = 0, mask = 0;
  bool ok = true;
  for (int shift = ((NBITS + 7) / 8 - 1) * 8; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += NT) hist[i] = 0;
    __syncthreads();
    visit([&](uint64_t key, uint64_t w) {
      if (w != 0 && (key & mask) == prefix)
        atomicAdd((unsigned long long*)&hist[(key >> shift) & 255], (unsigned long long)w);
    });
    __syncthreads();
    if (wid == 0) {
      uint64_t v[4];
      uint64_t s = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int bin = DESC ? 255 - (lane * 4 + q) : lane * 4 + q;
        v[q] = hist[bin];
        s += v[q];
      }
      const uint64_t incl = wave_incl_scan_u64(s, lane);
      const uint64_t before = incl - s;
      const uint64_t total = __shfl(incl, 63);
      if (before < target && target <= incl) {
        uint64_t acc = before;
        int digit = 0;
        uint64_t rem = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (acc < target && target <= acc + v[q] && rem == 0) {
            digit = DESC ? 255 - (lane * 4 + q) : lane * 4 + q;
            rem = target - acc;
          }
          acc += v[q];
        }
        m->bi[0] = digit;
        m->bu[0] = rem;
      }
      if (lane == 0 && total < target) {
        m->bi[0] = -1;
        m->bu[0] = 0;
      }
    }
    __syncthreads();
    const int digit = m->bi[0];
    const uint64_t rem = m->bu[0];
    __syncthreads();
    if (digit < 0) {
      ok = false;
      break;
    }
    target = rem;
    prefix |= (uint64_t)digit << shift;
    mask |= (uint64_t)0xFF << shift;
  }
  *found = ok;
  return ok ? prefix : 0;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, uint32_t bytes) {
  // gfx9 raw buffer: stride 0, num_records = bytes; reads past it return 0
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// ------------------------------------------------------------ history tables
// bitmap[w] bit b set <=> token 32w+b occurs in the row's history;
// wrank[w] = number of set bits before word w, so token t has slot
// wrank[t>>5] + popcount(bitmap[t>>5] below bit t&31); cnt[slot] = occurrences
// (16-bit halves of u32 words), tok[slot] = token.
struct Hist {
  uint32_t* bitmap;
  uint16_t* wrank;
  uint32_t* cnt2;
  uint32_t* tok;
};

__device__ __forceinline__ int slot_of(const Hist& h, int t) {
  const uint32_t w = h.bitmap[t >> 5];
  return (int)h.wrank[t >> 5] + __popc(w & ((1u << (t & 31)) - 1u));
}
__device__ __forceinline__ uint32_t count_of(const Hist& h, int s) {
  return (h.cnt2[s >> 1] >> ((s & 1) * 16)) & 0xFFFFu;
}
// number of slots of tokens < e (0 <= e <= V)
__device__ __forceinline__ int rank_below(const Hist& h, int e, int words, int U) {
  const int w = e >> 5;
  if (w >= words) return U;
  return (int)h.wrank[w] + __popc(h.bitmap[w] & ((1u << (e & 31)) - 1u));
}

// History ids of one row, loaded into registers at kernel start so that the table
// build does not wait on memory twice; ids past HR*NT are read again from memory.
// IdT = int32_t keeps each id in one register: negative ids (padding) become -1 and ids
// past 2^31 - 1 become INT32_MAX, which every vocabulary check still flags.
template <int HR, typename IdT = int64_t>
struct HistIds {
  IdT id[HR];
  int hl;
};

template <int NT, int HR, typename IdT>
__device__ __forceinline__ void load_history(const Params& p, int row, HistIds<HR, IdT>& hi) {
  hi.hl = 0;
  if (!p.has_pen) return;
  const int tid = threadIdx.x;
  const int64_t* hr = p.hist + (int64_t)row * p.hstride;
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(hr, (uint32_t)p.hstride * 8u);
#pragma unroll
  for (int j = 0; j < HR; ++j) {
    const v2i v = __builtin_amdgcn_raw_buffer_load_b64(rs, (uint32_t)(tid + j * NT) * 8u, 0, STREAM_CPOL);
    const int64_t g = (int64_t)(((uint64_t)(uint32_t)v.y << 32) | (uint32_t)v.x);
    if constexpr (sizeof(IdT) == 4)
      hi.id[j] = g < 0 ? -1 : (g > (int64_t)INT32_MAX ? INT32_MAX : (int32_t)g);
    else
      hi.id[j] = g;
  }
  int hl = p.hlens ? p.hlens[row] : p.hlen;
  hi.hl = max(0, min(hl, (int)p.hstride));
}

// Builds the tables; returns the number of slots (distinct in-vocabulary ids).  With
// counts false only the membership bitmap is built and 0 is returned.
template <int NT, int HR, bool SHARD = false, typename IdT = int64_t>
__device__ __forceinline__ int build_history(const Params& p, int row, const HistIds<HR, IdT>& hi, const Hist& h, Misc* m,
                                             bool counts = true) {
  // a vocabulary shard keeps the ids of its own range; ids past the whole vocabulary flag the row
  const int64_t id_off = SHARD ? p.voff : 0, id_lim = SHARD ? p.vfull : p.V;
  constexpr int NW = NT / 64;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int W = p.words;
  for (int i = tid; i < W; i += NT) h.bitmap[i] = 0;
  for (int i = tid; i < (p.ucap + 1) / 2; i += NT) h.cnt2[i] = 0;
  __syncthreads();
  const int hl = hi.hl;
  const int64_t* hr = p.hist + (int64_t)row * p.hstride;
  const int plen = p.plens ? p.plens[row] : 0;  // entries [0, plen) belong to the prompt
  int bad = 0;
#pragma unroll
  for (int j = 0; j < HR; ++j) {
    const int idx = tid + j * NT;
    if (idx < hl) {
      const int64_t g = hi.id[j], id = g - id_off;
      if (id >= 0 && id < p.V) atomicOr(&h.bitmap[id >> 5], 1u << (id & 31));
      else if (g >= id_lim) bad = 1;
    }
  }
  for (int idx = tid + HR * NT; idx < hl; idx += NT) {
    const int64_t g = hr[idx], id = g - id_off;
    if (id >= 0 && id < p.V) atomicOr(&h.bitmap[id >> 5], 1u << (id & 31));
    else if (g >= id_lim) bad = 1;
  }
  if (bad) atomicOr(&m->status, ST_BAD_HISTORY);
  __syncthreads();
  if (!counts) return 0;
  const int per = (W + NT - 1) / NT;
  const int b = tid * per, e = min(b + per, W);
  int s = 0;
  for (int i = b; i < e; ++i) s += __popc(h.bitmap[i]);
  const int incl = (int)wave_incl_scan_u32((uint32_t)s);
  if (lane == 63) m->ri[wid] = incl;
  __syncthreads();
  // lane w reads wave w's count; their scan gives the slots before this wave and U
  const int wtot = (int)wave_incl_scan_u32(lane < NW ? (uint32_t)m->ri[lane] : 0u);
  const int off = wid > 0 ? __builtin_amdgcn_readlane(wtot, wid - 1) : 0;
  const int U = __builtin_amdgcn_readlane(wtot, NW - 1);
  int run = off + incl - s;
  for (int i = b; i < e; ++i) {
    h.wrank[i] = (uint16_t)run;
    run += __popc(h.bitmap[i]);
  }
  __syncthreads();
  auto count_id = [&](int64_t g, int idx) {
    const int64_t id = g - id_off;
    if (id >= 0 && id < p.V) {
      const int slot = slot_of(h, (int)id);
      if (idx >= plen) atomicAdd(&h.cnt2[slot >> 1], 1u << ((slot & 1) * 16));
      h.tok[slot] = (uint32_t)id;
    }
  };
#pragma unroll
  for (int j = 0; j < HR; ++j)
    if (tid + j * NT < hl) count_id(hi.id[j], tid + j * NT);
  for (int idx = tid + HR * NT; idx < hl; idx += NT) count_id(hr[idx], idx);
  __syncthreads();
  return U;
}

// ------------------------------------------------------------ streaming loads
template <typename TIn, int G>
struct Raw {
  static constexpr int WORDS = G * (int)sizeof(TIn) / 4;
  uint32_t w[WORDS];
};

template <typename TIn, int G, bool VEC, int CPOL = STREAM_CPOL>
__device__ __forceinline__ void load_group(Raw<TIn, G>& r, __amdgpu_buffer_rsrc_t rs, int base) {
  constexpr int WORDS = Raw<TIn, G>::WORDS;
  const uint32_t off = (uint32_t)base * (uint32_t)sizeof(TIn);
  if constexpr (VEC && WORDS == 4) {
    const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, CPOL);
    r.w[0] = (uint32_t)v.x;
    r.w[1] = (uint32_t)v.y;
    r.w[2] = (uint32_t)v.z;
    r.w[3] = (uint32_t)v.w;
  } else if constexpr (VEC && WORDS == 8) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rs, off + 16 * h, 0, CPOL);
      r.w[4 * h] = (uint32_t)v.x;
      r.w[4 * h + 1] = (uint32_t)v.y;
      r.w[4 * h + 2] = (uint32_t)v.z;
      r.w[4 * h + 3] = (uint32_t)v.w;
    }
  } else if constexpr (VEC && WORDS == 2) {
    const v2i v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, CPOL);
    r.w[0] = (uint32_t)v.x;
    r.w[1] = (uint32_t)v.y;
  } else if constexpr (sizeof(TIn) == 4) {
#pragma unroll
    for (int j = 0; j < G; ++j) r.w[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, off + 4 * j, 0, CPOL);
  } else {
#pragma unroll
    for (int i = 0; i < WORDS; ++i) {
      const uint32_t lo = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off + 4 * i, 0, CPOL);
      const uint32_t hi = (uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, off + 4 * i + 2, 0, CPOL);
      r.w[i] = lo | (hi << 16);
    }
  }
}

template <typename TIn>
__device__ __forceinline__ float load_one(__amdgpu_buffer_rsrc_t rs, int idx) {
  if constexpr (sizeof(TIn) == 4)
    return __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, (uint32_t)idx * 4u, 0, 0));
  else
    return bf16_to_f32((uint16_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (uint32_t)idx * 2u, 0, 0));
}

template <typename TIn, int G>
__device__ __forceinline__ void unpack(const Raw<TIn, G>& r, float (&x)[G]) {
  if constexpr (sizeof(TIn) == 4) {
#pragma unroll
    for (int j = 0; j < G; ++j) x[j] = __uint_as_float(r.w[j]);
  } else {
#pragma unroll
    for (int j = 0; j < G / 2; ++j) {
      x[2 * j] = bf16_lo(r.w[j]);
      x[2 * j + 1] = bf16_hi(r.w[j]);
    }
  }
}

// z for G logits at [base, base+G).  History tokens and (TAIL) indices >= V become
// -inf; the exact values of history tokens come from the batch gather instead.  `bitmap`
// holds the history bits of ids from bit_off on (a multiple of 32).
template <int G, bool TAIL>
__device__ __forceinline__ void make_z(const float (&x)[G], int base, const Params& p,
                                       const uint32_t* bitmap, float (&z)[G], int& bad, int bit_off = 0) {
  uint32_t pen = 0;
  if (p.has_pen && (!TAIL || base < p.V))
    pen = (bitmap[(base - bit_off) >> 5] >> (base & 31)) & ((1u << G) - 1u);
  // a non-finite logit outside the history and inside the row flags the row (history ids are
  // checked where their penalized value is formed; ids past the row read 0)
  auto check = [&](const float (&v)[G]) {
#pragma unroll
    for (int j = 0; j < G; ++j)
      if ((!TAIL || base + j < p.V) && !((pen >> j) & 1u) && !isfinite(v[j])) bad = 1;
  };
  if (p.unit_T) {
    // x / 1 = x for every x: one class test per logit, the exact check only when one fails
    bool nf = false;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      z[j] = x[j];
      nf |= __builtin_amdgcn_classf(x[j], 0x207);  // NaN or an infinity
    }
    if (nf) check(z);
  } else {
    // 2^-100 <= |x| < 2^100: the three-operation division is IEEE-exact there (checked
    // exhaustively on the host); outside it, IEEE division.
    uint32_t lo = 0xFFFFFFFFu, hi = 0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const uint32_t a = __float_as_uint(x[j]) & 0x7FFFFFFFu;
      lo = min(lo, a);
      hi = max(hi, a);
    }
    if (p.fast_div && lo >= 0x0D800000u && hi < 0x71800000u) {
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const float q = x[j] * p.rT;
        const float e = __builtin_fmaf(-q, p.T, x[j]);
        z[j] = __builtin_fmaf(e, p.rT, q);
      }
    } else {
#pragma unroll
      for (int j = 0; j < G; ++j) z[j] = x[j] / p.T;
      check(z);
    }
  }
  if (p.has_pen) {
    // history ids read -inf here: a signed one-bit field gives an all-ones or zero mask and
    // v_bfi_b32 picks by it (a compare and v_cndmask through VCC would cost wait states)
    const uint32_t ninf = NEG_INF_BITS;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const uint32_t msk = (uint32_t)__builtin_amdgcn_sbfe((int)pen, j, 1);
      uint32_t r;
      asm("v_bfi_b32 %0, %1, %2, %3" : "=v"(r) : "v"(msk), "s"(ninf), "v"(__float_as_uint(z[j])));
      z[j] = __uint_as_float(r);
    }
  }
  if (TAIL) {
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (base + j >= p.V) z[j] = NEG_INF;
  }
}

// Adjacent floats (IEEE order; -0 is treated as +0; infinities and NaN map to themselves
// where no neighbour exists).
__device__ __forceinline__ float next_up(float x) {
  if (x != x) return x;
  uint32_t b = __float_as_uint(x);
  if (b == 0x80000000u) b = 0;
  if ((int32_t)b >= 0) {
    if (b == 0x7F800000u) return x;
    return __uint_as_float(b + 1u);
  }
  return __uint_as_float(b - 1u);
}
__device__ __forceinline__ float next_down(float x) { return -next_up(-x); }

// Smallest float x with RN(x / T) > t.  RN(x / T) is non-decreasing in x, so these x
// form an up-set; its least element is reached by stepping from t*T.  If the steps
// run out the result errs low, which only admits more candidates.
__device__ __forceinline__ float x_above(float t, const Params& p) {
  if (!(t > NEG_INF)) return -__FLT_MAX__;
  if (!(t < __builtin_huge_valf())) return __builtin_huge_valf();
  float x = t * p.T;
  for (int i = 0; i < 8 && x / p.T > t; ++i) x = next_down(x);
  if (x / p.T > t) x = x - __builtin_fmaf(fabsf(x), 0x1p-10f, 0x1p-126f);
  for (int i = 0; i < 8 && !(x / p.T > t); ++i) x = next_up(x);
  return x;
}

// Raw-logit threshold of the TOPK filter: x passes iff RN(x/T) > tau and RN(x/T) >= bnd.
__device__ __forceinline__ float x_threshold(float tau, float bnd, const Params& p) {
  return fmaxf(x_above(tau, p), x_above(next_down(bnd), p));
}

// RN(x / T): the three-operation scheme inside the range where it is exact (the guard of
// make_z), IEEE division outside it.
__device__ __forceinline__ float div_T(float x, const Params& p) {
  const uint32_t a = __float_as_uint(x) & 0x7FFFFFFFu;
  if (p.fast_div && a >= 0x0D800000u && a < 0x71800000u) {
    const float q = x * p.rT;
    return __builtin_fmaf(__builtin_fmaf(-q, p.T, x), p.rT, q);
  }
  return x / p.T;
}

// exact processed logit of a history token from its raw logit
__device__ __forceinline__ float pen_z(float x, uint32_t c, const Params& p) {
  return penalize(x, c, p) / p.T;
}

// An empty instruction that reads v.  Where a path never uses a loaded value, the
// compiler's wait analysis still counts the load as pending on that path and makes the
// next write of the register (the next batch's load) wait for every older load; reading
// the value here ends that on every path.
template <typename T>
__device__ __forceinline__ void landed(T v) {
  asm volatile("" ::"v"(v));
}
template <int HR, typename IdT>
__device__ __forceinline__ void landed(const HistIds<HR, IdT>& hi) {
#pragma unroll
  for (int j = 0; j < HR; ++j) landed(hi.id[j]);
}

// Pipelined row stream.  `setup()` builds the history tables while the first batch
// is in flight and returns the slot count.  `batch(t0, nt, R, s0, n, gx)` processes
// tiles [t0, t0+PF) (TILE = NT*G elements each; tiles >= nt read as zeros) from the
// raw registers R, together with the history slots [s0, s0+n) whose tokens lie in
// those tiles: thread i holds the raw logit of slot s0+i in gx (for i < NT).
// LOWERING: the caller meets history tokens in the stream itself when p.pen_lowers is
// set, and the gather is off then (a compile-time switch: an extra runtime flag costs
// full_kernel the scalar registers that keep it at two workgroups per CU).
template <typename TIn, int G, int NT, bool VEC, bool LOWERING, int CPOL = STREAM_CPOL, int PF = dsv41::sampler::PF,
          class Setup, class Batch>
__device__ __forceinline__ void stream_row(const Params& p, __amdgpu_buffer_rsrc_t rs, const Hist& h,
                                           Setup setup, Batch batch) {
  constexpr int TILE = NT * G;
  const int tid = threadIdx.x;
  const int nt = (p.V + TILE - 1) / TILE;
  Raw<TIn, G> A[PF], B[PF];
#pragma unroll
  for (int k = 0; k < PF; ++k) load_group<TIn, G, VEC, CPOL>(A[k], rs, k * TILE + tid * G);
  const int U = setup();
  auto gather = [&](int t0, int& s0, int& n) -> float {
    if (!p.has_pen || (LOWERING && p.pen_lowers)) {
      s0 = 0;
      n = 0;
      return 0.0f;
    }
    s0 = rank_below(h, min(t0 * TILE, p.V), p.words, U);
    n = rank_below(h, min((t0 + PF) * TILE, p.V), p.words, U) - s0;
    return tid < n ? load_one<TIn>(rs, (int)h.tok[s0 + tid]) : 0.0f;
  };
  int sA, nA, sB = 0, nB = 0;
  float gA = gather(0, sA, nA), gB = 0.0f;
  for (int t0 = 0; t0 < nt; t0 += 2 * PF) {
#pragma unroll
    for (int k = 0; k < PF; ++k) load_group<TIn, G, VEC, CPOL>(B[k], rs, (t0 + PF + k) * TILE + tid * G);
    gB = gather(t0 + PF, sB, nB);
    batch(t0, nt, A, sA, nA, gA);
    if (t0 + PF >= nt) break;
#pragma unroll
    for (int k = 0; k < PF; ++k) load_group<TIn, G, VEC, CPOL>(A[k], rs, (t0 + 2 * PF + k) * TILE + tid * G);
    gA = gather(t0 + 2 * PF, sA, nA);
    batch(t0 + PF, nt, B, sB, nB, gB);
  }
}

// Conservative fp32 lower bound of mrun + log(min_p) (lmin_f = log(min_p) rounded
// down): elements below it can never pass min-p, because the row maximum is at
// least mrun.  The subtracted margin exceeds both roundings of the float sums.
__device__ __forceinline__ float minp_bound_f(float mrun, float lmin_f) {
  if (!(mrun > NEG_INF) || !(lmin_f > NEG_INF)) return NEG_INF;
  const float t = mrun + lmin_f;
  return t - __builtin_fmaf(fabsf(t), 0x1p-20f, 0x1p-120f);
}

__device__ __forceinline__ void write_result(const Params& p, int row, Misc* m, int64_t id,
                                             float lp, int kept) {
  const int st = m->status;
  if (st & ST_NONFINITE) {
    p.out_ids[row] = -1;
    if (p.out_lp) p.out_lp[row] = __builtin_nanf("");
    if (p.out_kept) p.out_kept[row] = 0;
  } else {
    p.out_ids[row] = id;
    if (p.out_lp) p.out_lp[row] = lp;
    if (p.out_kept) p.out_kept[row] = kept;
  }
  p.out_status[row] = st;
}

// A row's maximum and total over the gathered slice states, in slice order (fp64); the
// draw kernels and the finish kernel evaluate the same expression on the same states.
__device__ __forceinline__ double slice_weight(const dsv41_full_state& st, float M) {
  return st.max_z > NEG_INF ? st.mass * exp((double)st.max_z - (double)M) : 0.0;
}
__device__ __forceinline__ void combine_states(const dsv41_full_state* states, int n_shards, int nrows, int row,
                                               float& M, double& S) {
  M = NEG_INF;
  for (int s = 0; s < n_shards; ++s) M = fmaxf(M, states[(int64_t)s * nrows + row].max_z);
  S = 0.0;
  for (int s = 0; s < n_shards; ++s) S += slice_weight(states[(int64_t)s * nrows + row], M);
}

__device__ __forceinline__ float row_uniform(const Params& p, int row, Misc* m) {
  if (p.greedy) return 0.0f;
  const float u = p.uniforms[row];
  if (!(u >= 0.0f && u < 1.0f)) {
    atomicOr(&m->status, ST_BAD_UNIFORM);
    return 0.0f;
  }
  return u;
}

template <typename TIn>
__device__ __forceinline__ const TIn* row_ptr(const Params& p, int row) {
  return reinterpret_cast<const TIn*>(p.logits) + (int64_t)row * p.lstride;
}

__device__ __forceinline__ Hist hist_tables(unsigned char* smem, const Layout& L) {
  Hist h;
  h.bitmap = reinterpret_cast<uint32_t*>(smem + L.bitmap);
  h.wrank = reinterpret_cast<uint16_t*>(smem + L.wrank);
  h.cnt2 = reinterpret_cast<uint32_t*>(smem + L.cnt);
  h.tok = reinterpret_cast<uint32_t*>(smem + L.tok);
  return h;
}

// Each lane's 16-lane row total of v (fp64, by the same DPP steps).
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)b, CTRL, 0xF, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(b >> 32), CTRL, 0xF, 0xF, true);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double row_sum_f64(double v) {
  v += dpp_f64<0xB1>(v);
  v += dpp_f64<0x4E>(v);
  v += dpp_f64<0x124>(v);
  v += dpp_f64<0x128>(v);
  return v;
}
// floor(w * g / 2^43) for w < 2^52 and an integer-valued g <= 2^43 (a mass_ff result).
__device__ __forceinline__ uint64_t scale_mass(uint64_t w, float g) {
  return (uint64_t)(((unsigned __int128)w * (uint64_t)g) >> 43);
}

// Statistics of one wave span of 64 G processed logits (lane l holds z for ids l G ..
// l G + G - 1 of the span): mc = the maximum of the lane's 256-id mass chunk (the span, or
// its half: lanes 0-31 and 32-63); rs4 = the lane's 16-lane row total of the masses
// floor(2^43 exp32(z - mc)), integers of at most 2^43, so the fp64 sums are exact in any
// order (a chunk's total is below 2^51).
template <int G, bool MASSES = true>
__device__ __forceinline__ void span_stats(const float (&z)[G], float& mc, double& rs4) {
  static_assert(G == 4 || G == 8, "a mass chunk is the span (G 4) or its half (G 8)");
  float mx = z[0];
#pragma unroll
  for (int j = 1; j < G; ++j) mx = fmaxf(mx, z[j]);
  mx = pair_max_q(row_max_q(__builtin_canonicalizef(mx)));
  mc = G == 4 ? halves_max_q(mx) : mx;
  if constexpr (MASSES) {
    double qd = (double)mass_ff(z[0], mc);
#pragma unroll
    for (int j = 1; j < G; ++j) qd += (double)mass_ff(z[j], mc);
    rs4 = row_sum_f64(qd);
  }
}

__device__ __forceinline__ uint64_t rl_u64(uint64_t v, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ double rl_d(double v, int lane) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), lane);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}

// A small batch spread over the GPU: workgroup b takes slice b % n_slices (slice_w wave
// spans of 64 G ids) of row b / n_slices, one span per wave at a time, and writes the span
// statistics full_kernel's stream forms (span_stats on the same z), so full_kernel<...,
// PRE> finishes each row with the values and the order of the one-workgroup kernel: the
// same ids and log-probs, bit for bit.  With penalties the slice first marks the history
// ids of its own range in an LDS bitmap (2 G words per span) from the row's history list,
// so its history tokens read -inf as in the stream; their penalized values are the
// finishing kernel's.
constexpr int PRE_NT = 256;
template <typename TIn, int G, bool VEC, bool MASSES = true>
__global__ __launch_bounds__(PRE_NT) void full_slice_kernel(Params p) {
  constexpr int NW = PRE_NT / 64;
  extern __shared__ __align__(16) unsigned char smem[];
  const int row = blockIdx.x / p.n_slices, sl = blockIdx.x % p.n_slices;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int NC = n_chunks<G>(p.V), NE = n_mass_chunks(p.V);
  const int c1 = min((sl + 1) * p.slice_w, NC);
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(row_ptr<TIn>(p, row), (uint32_t)p.V * (uint32_t)sizeof(TIn));
  float* oem = p.pre_em + (int64_t)row * NE;
  uint64_t* ow = p.pre_w + (int64_t)row * NE;
  int bad = 0;
  int c = sl * p.slice_w + wid;
  Raw<TIn, G> A;
  if (c < c1) load_group<TIn, G, VEC, FULL_CPOL>(A, rs, c * 64 * G + lane * G);
  uint32_t* sbm = reinterpret_cast<uint32_t*>(smem);  // history bits of the slice's ids, from v0 on
  const int v0 = sl * p.slice_w * 64 * G;
  if (p.has_pen) {
    const int words = p.slice_w * 2 * G;
    for (int i = tid; i < words; i += PRE_NT) sbm[i] = 0;
    __syncthreads();
    const int64_t* hr = p.hist + (int64_t)row * p.hstride;
    const int hl = max(0, min(p.hlens ? p.hlens[row] : p.hlen, (int)p.hstride));
    const int64_t v1 = min((int64_t)c1 * 64 * G, (int64_t)p.V);
    for (int i = tid; i < hl; i += PRE_NT) {
      const int64_t g = hr[i];
      if (g >= v0 && g < v1) atomicOr(&sbm[(int)(g - v0) >> 5], 1u << ((int)(g - v0) & 31));
    }
    __syncthreads();
  }
  while (c < c1) {  // uniform per wave; the next span's load is in flight meanwhile
    const int cn = c + NW;
    Raw<TIn, G> B;
    if (cn < c1) load_group<TIn, G, VEC, FULL_CPOL>(B, rs, cn * 64 * G + lane * G);
    const int base = c * 64 * G + lane * G;
    float x[G], z[G];
    unpack(A, x);
    make_z<G, true>(x, base, p, sbm, z, bad, v0);  // history ids and ids past V read -inf
    float mc;
    double rs4 = 0.0;
    span_stats<G, MASSES>(z, mc, rs4);
    const int e = c * (64 * G / MASS_CHUNK) + (G == 4 ? 0 : (lane >> 5));
    if ((G == 4 ? lane : (lane & 31)) == 0 && e < NE) oem[e] = mc;
    if constexpr (MASSES) {
      const double r0 = rl_d(rs4, 0), r1 = rl_d(rs4, 16), r2 = rl_d(rs4, 32), r3 = rl_d(rs4, 48);
      if (G == 4) {
        if (lane == 0 && e < NE) ow[e] = (uint64_t)((r0 + r1) + (r2 + r3));
      } else {
        if (lane == 0 && e < NE) ow[e] = (uint64_t)(r0 + r1);
        if (lane == 32 && e < NE) ow[e] = (uint64_t)(r2 + r3);
      }
    }
    if (cn < c1) A = B;
    c = cn;
  }
  bad = __syncthreads_or(bad);
  if (tid == 0) p.pre_st[(int64_t)row * p.n_slices + sl] = bad ? ST_NONFINITE : 0;
}

// ====================================================================== FULL
// No truncation: kept set = whole vocabulary.  Span c = [c*64G, (c+1)*64G) is one wave's
// span of one tile; the exact masses of its one or two 256-id chunks go to LDS.
// fp32 rows of the draws that form masses take 8 logits per lane (two 16-byte loads) in
// batches of one tile, so that each wave span's reductions spread over 8 logits; the two
// tiles in flight (128 KiB per CU at two workgroups) cover the latency of this ALU-bound
// stream.  The massless argmax and the spread small batches keep 4 per lane,
// whose loads read whole contiguous kilobytes (measured faster there).
template <typename TIn, int G>
constexpr int full_pf() { return sizeof(TIn) * G > 16 ? 1 : PF; }
template <typename TIn, int G, bool VEC, int DRAW, bool PRE = false>
__global__ __launch_bounds__(FULL_NT, sizeof(TIn) == 4 ? 8 : 1) void full_kernel(Params p) {
  constexpr int NT = FULL_NT, NW = NT / 64, HR = 4;
  extern __shared__ __align__(16) unsigned char smem[];
  const Layout L = make_layout<MODE_FULL, G>(p.V, p.words, p.ucap, 0);
  Misc* m = reinterpret_cast<Misc*>(smem + L.misc);
  const Hist h = hist_tables(smem, L);
  float* penz = reinterpret_cast<float*>(smem + L.penx);
  const int NC = n_chunks<G>(p.V);
  const int NE = n_mass_chunks(p.V);
  // exact masses of the 256-id chunks: during the stream fp64 sums of integers below 2^51
  // (exact in any order), then the u64 chunk weights
  uint64_t* cq = reinterpret_cast<uint64_t*>(smem + L.mode0);
  double* cqd = reinterpret_cast<double*>(cq);
  float* em = reinterpret_cast<float*>(cq + NE);  // 256-id chunk maxima over ids outside the history
  // the maximum of wave span c: one 256-id chunk (G = 4) or two (G = 8)
  auto span_max = [&](int c) {
    if (G == 4) return em[c];
    return 2 * c + 1 < NE ? fmaxf(em[2 * c], em[2 * c + 1]) : em[2 * c];
  };
  constexpr bool SLICE = DRAW == DRAW_STATE || DRAW == DRAW_SHARD_CDF || DRAW == DRAW_SHARD_RACE ||
                         DRAW == DRAW_SHARD_MASS;
  // Every draw takes exact fixed-point masses (see below) in the same pass as the maximum:
  // w_i = floor(2^43 exp32(z_i - m_c)) against the maximum m_c of the token's 256-id chunk,
  // summed exactly per chunk.  The inverse-CDF draws place their target in them.
  constexpr bool PLACES = DRAW == DRAW_CDF || DRAW == DRAW_SHARD_CDF;
  // a greedy draw whose log-prob nobody asked for needs the maxima alone
  constexpr bool MASSES = DRAW != DRAW_ARGMAX;
  static_assert(64 * G == MASS_CHUNK || 64 * G == 2 * MASS_CHUNK, "a wave span holds one or two mass chunks");

  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const TIn* src = row_ptr<TIn>(p, row);
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(src, (uint32_t)p.V * (uint32_t)sizeof(TIn));
  constexpr int TILE = NT * G;
  int bad = 0;
  int U = 0;
  // This thread's running maximum of chunk maxima and history z.  bf16 rows (one workgroup
  // per CU, whose serial phases nothing hides) keep it during the stream; fp32 rows run at
  // the 64-register cap, where one more live register costs the stream more than reading
  // the tables afterwards does.
  constexpr bool RUN_MAX = PRE || sizeof(TIn) == 2;
  float lmax = NEG_INF;
  if constexpr (PRE) {
    // the span statistics full_slice_kernel formed; with penalties, the history tables and
    // the history tokens' penalized z, which the slices left out
    HistIds<HR> hi;
    load_history<NT, HR>(p, row, hi);
    if (tid == 0) m->status = 0;
    const float* pem = p.pre_em + (int64_t)row * NE;
    const uint64_t* pw = p.pre_w + (int64_t)row * NE;
    for (int e = tid; e < NE; e += NT) {
      em[e] = pem[e];
      lmax = fmaxf(lmax, em[e]);
      if constexpr (MASSES) cqd[e] = (double)pw[e];
    }
    for (int s = tid; s < p.n_slices; s += NT) bad |= p.pre_st[(int64_t)row * p.n_slices + s];
    __syncthreads();  // status cleared before any thread sets a bit
    if (p.has_pen) {
      U = build_history<NT, HR>(p, row, hi, h, m);
      for (int s = tid; s < U; s += NT) {
        const float z = pen_z(load_one<TIn>(rs, (int)h.tok[s]), count_of(h, s), p);
        if (!isfinite(z)) bad = 1;
        penz[s] = z;
        lmax = fmaxf(lmax, z);
      }
    }
    landed(hi);  // the ids are read under conditions; end their loads on every path
  } else {
  HistIds<HR> hi;
  load_history<NT, HR>(p, row, hi);
  constexpr int FPF = full_pf<TIn, G>();
  stream_row<TIn, G, NT, VEC, false, FULL_CPOL, FPF>(
      p, rs, h,
      [&]() {
        if (tid == 0) m->status = 0;
        if constexpr (MASSES)
          for (int e = tid; e < NE; e += NT) cq[e] = 0;
        // the history build's first barrier also publishes the cleared status and masses
        if (p.has_pen) U = build_history<NT, HR, SLICE>(p, row, hi, h, m);
        else __syncthreads();
        landed(hi);  // the ids are read under conditions; end their loads on every path
        return U;
      },
      [&](int t0, int nt, Raw<TIn, G>(&R)[FPF], int s0, int n, float gx) {
#pragma unroll
        for (int k = 0; k < FPF; ++k) {
          const int t = t0 + k;
          if (t < nt) {
            const int base = t * TILE + tid * G;
            float x[G], z[G];
            unpack(R[k], x);
            if ((t + 1) * TILE <= p.V) make_z<G, false>(x, base, p, h.bitmap, z, bad);
            else make_z<G, true>(x, base, p, h.bitmap, z, bad);
            float mc;
            double rs4 = 0.0;
            span_stats<G, MASSES>(z, mc, rs4);
            if constexpr (RUN_MAX) lmax = fmaxf(lmax, mc);
            // the lane's 256-id chunk: the span, or its half for G = 8
            const int e = (t * TILE + wid * 64 * G) / MASS_CHUNK + (G == 4 ? 0 : (lane >> 5));
            if ((G == 4 ? lane : (lane & 31)) == 0 && e < NE) em[e] = mc;
            // rows 0 + 1 (and 2 + 3) are one chunk: each row's lane 0 adds its total
            if constexpr (MASSES)
              if ((lane & 15) == 0 && e < NE) atomicAdd(&cqd[e], rs4);
          }
        }
        for (int i = tid; i < n; i += NT) {
          const int s = s0 + i;
          const float x = i == tid ? gx : load_one<TIn>(rs, (int)h.tok[s]);
          const float z = pen_z(x, count_of(h, s), p);
          if (!isfinite(z)) bad = 1;
          penz[s] = z;
          if constexpr (RUN_MAX) lmax = fmaxf(lmax, z);
        }
      });
  }
  if (bad) atomicOr(&m->status, ST_NONFINITE);
  if constexpr (!RUN_MAX) {
    __syncthreads();
    for (int s = tid; s < U; s += NT) lmax = fmaxf(lmax, penz[s]);
    for (int c = tid; c < NE; c += NT) lmax = fmaxf(lmax, em[c]);
  }
  // the row maximum over the chunk maxima and the history tokens' z (the barriers inside
  // also publish the stream's LDS tables)
  const float M = block_max<NT>(lmax, m);

  // The draws use 2^-43 fixed-point masses, exact integers, so neither the drawn id nor
  // the reported log-prob depends on the order of any reduction.  The row (or slice) is cut
  // into 256-id chunks.  In the stream, an id outside the history got
  // w_i = floor(2^43 exp32(z_i - m_c)) against its chunk's maximum m_c over such ids, and
  // cqd[c] = W_c = sum w_i.  With the row's maximum Mref known (a slice of a sharded
  // inverse-CDF draw: the maximum over all slices), the chunk weighs
  //   Q_c = floor(W_c g_c / 2^43),  g_c = floor(2^43 exp32(m_c - Mref)),
  // plus the history ids' masses floor(2^43 exp32(z_h - Mref)) (their slots are in id order,
  // so a chunk's slots are one run, summed by one thread); the oracle defines the same
  // integers.  S = sum Q_c is the row's total: every draw, the replay included, reports
  // lp = (z_tok - M) - log(S 2^-43), so DRAW_REPLAY of a drawn token returns the same float
  // bit for bit.
  constexpr bool SHARDED = DRAW == DRAW_SHARD_CDF || DRAW == DRAW_SHARD_MASS;
  float Mref = M;
  if constexpr (SHARDED) {
    double Sg;
    combine_states(p.sh_states, p.n_shards, p.nrows, row, Mref, Sg);
  }
  // The inverse-CDF draws need the uniform before the masses are scanned; a slice of a
  // sharded draw learns here whether its masses hold the target at all.
  const float u = PLACES ? row_uniform(p, row, m) : 0.0f;
  uint64_t tq = 0;  // the draw's target in this workgroup's masses
  if constexpr (DRAW == DRAW_SHARD_CDF) {
    // Every slice finds, from the same gathered masses, the slice whose masses hold the
    // target; only that one places the token, against the target less the masses before it.
    uint64_t Sall = 0;
    for (int s = 0; s < p.n_shards; ++s) Sall += p.sh_masses[(int64_t)s * p.nrows + row];
    const uint64_t t = draw_target(u, Sall);
    uint64_t acc = 0;
    int owner = -1;
    for (int s = 0; s < p.n_shards; ++s) {
      const uint64_t q = p.sh_masses[(int64_t)s * p.nrows + row];
      if (owner < 0 && t < acc + q) {
        owner = s;
        tq = t - acc;
      }
      acc += q;
    }
    if (owner != p.shard_index) {  // uniform over the workgroup
      if (tid == 0) p.sh_out_picks[row] = dsv41_full_pick{-1, NEG_INF, -1.0f};
      return;
    }
  }
  // Thread t forms the masses of the contiguous run of chunks [cb, ce) (one chunk per
  // thread up to 1024 chunks) and their sum `own`; a block scan of the sums gives every
  // thread S and its run's exclusive prefix `before`.  The inverse-CDF target t = (S U) >> 32
  // lies in the first chunk whose cumulative Q exceeds it, which the one thread whose run
  // holds t records; inside that chunk the id boundaries in Q units are
  // floor(prefix(w) g_c / 2^43) + prefix(history masses), in vocabulary order.
  uint64_t S = 0;
  if constexpr (DRAW != DRAW_SHARD_RACE && MASSES) {  // the race over slices takes the gathered states
    const int crun = (NE + NT - 1) / NT;
    const int cb = min(tid * crun, NE), ce = min(cb + crun, NE);
    uint64_t own = 0;
    for (int c = cb; c < ce; ++c) {
      uint64_t q = scale_mass((uint64_t)cqd[c], mass_ff(em[c], Mref));
      if (p.has_pen) {
        const int s1 = rank_below(h, min((c + 1) * MASS_CHUNK, p.V), p.words, U);
        for (int s = rank_below(h, c * MASS_CHUNK, p.words, U); s < s1; ++s) q += mass_of(penz[s], Mref);
      }
      cq[c] = q;
      own += q;
    }
    if (PLACES && tid == 0) m->bi[0] = -1;  // no chunk holds the target (no mass at all)
    const uint64_t incl = wave_incl_scan_u64(own, lane);
    if (lane == 63) m->ru[wid] = incl;
    __syncthreads();
    // lane w reads wave w's total; their scan gives S and the totals of the waves before
    // this one (one read per lane: a loop over the totals keeps them all in registers)
    const uint64_t wtot = wave_incl_scan_u64(lane < NW ? m->ru[lane] : 0, lane);
    S = rl_u64(wtot, NW - 1);
    uint64_t before = incl - own + (wid > 0 ? rl_u64(wtot, wid - 1) : 0);
    if constexpr (PLACES) {
      if constexpr (DRAW == DRAW_CDF) tq = draw_target(u, S);
      if (before <= tq && tq < before + own) {
        for (int c = cb; c < ce; ++c) {  // this thread's own chunk masses
          if (tq < before + cq[c]) {
            m->bi[0] = c;
            m->bu[0] = tq - before;
            break;
          }
          before += cq[c];
        }
      }
      __syncthreads();
    }
  }
  auto row_lp = [&](float ztok, uint64_t total) {
    return (float)(((double)ztok - (double)M) - log((double)total * 0x1p-43));
  };

  if constexpr (DRAW == DRAW_REPLAY) {
    // the given token's processed log-prob (a separate instantiation, like the race)
    if (tid == 0) {
      const int64_t tok = p.replay[row];
      float lp = __builtin_nanf("");
      if (tok >= 0 && tok < p.V) {
        const int t = (int)tok;
        const bool pen = p.has_pen && ((h.bitmap[t >> 5] >> (t & 31)) & 1u);
        const float ztok = pen ? penz[slot_of(h, t)] : load_one<TIn>(rs, t) / p.T;
        lp = row_lp(ztok, S);
      } else {
        m->status |= ST_BAD_TARGET;
      }
      write_result(p, row, m, tok, lp, p.V);
    }
    return;
  }

  if ((DRAW == DRAW_RACE || DRAW == DRAW_SHARD_RACE) && !p.greedy) {
    // (a separate instantiation: the race's registers would cost the inverse-CDF draw occupancy)
    // Exponential race: the token is argmax_i p_i / E_i with p_i = exp(log_softmax(z)_i),
    // each step in fp32 as torch forms it (log_softmax = z - (max + log(sum)), exp,
    // division), first index on ties.  This is torch.multinomial(p, 1) on the CPU fed the
    // same E (its draw is exponential_ followed by argmax(p / E)); only the order of the
    // sum differs, which moves every p by the same factor and can reorder only ratios
    // within an ulp of each other.
    float Mr = M;  // the row's maximum (a slice: over all slices)
    double Sr;     // the row's sum of exp(z - Mr)
    if constexpr (DRAW == DRAW_SHARD_RACE) {
      combine_states(p.sh_states, p.n_shards, p.nrows, row, Mr, Sr);
    } else {
      Sr = (double)S * 0x1p-43;
    }
    const float lsum = Mr + logf((float)Sr);
    const float* erow = p.exps + (int64_t)row * p.estride;
    const __amdgpu_buffer_rsrc_t re = row_rsrc(erow, (uint32_t)p.V * 4u);
    float best = -1.0f;
    int bidx = 0x7FFFFFFF;
    auto offer = [&](float z, float ev, int idx) {
      const float pr = expf(z - lsum);
      const float r = pr / ev;
      if (r > best || (r == best && idx < bidx)) {
        best = r;
        bidx = idx;
      }
    };
    const int nt = (p.V + TILE - 1) / TILE;
    for (int t = 0; t < nt; ++t) {
      const int base = t * TILE + tid * G;
      Raw<TIn, G> r;
      load_group<TIn, G, VEC, FULL_CPOL>(r, rs, base);
      Raw<float, G> er;
      load_group<float, G, false, FULL_CPOL>(er, re, base);
      float x[G], z[G];
      unpack(r, x);
      int dummy = 0;
      make_z<G, true>(x, base, p, h.bitmap, z, dummy);  // history tokens and the tail read -inf
#pragma unroll
      for (int j = 0; j < G; ++j)
        if (base + j < p.V && z[j] > NEG_INF) offer(z[j], __uint_as_float(er.w[j]), base + j);
    }
    for (int s = tid; s < U; s += NT) offer(penz[s], erow[h.tok[s]], (int)h.tok[s]);
    // fixed-order argmax: waves by shuffles, then waves in turn
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ob = __shfl_xor(best, o);
      const int oi = __shfl_xor(bidx, o);
      if (ob > best || (ob == best && oi < bidx)) {
        best = ob;
        bidx = oi;
      }
    }
    if (lane == 0) {
      m->rf[wid] = best;
      m->ri[wid] = bidx;
    }
    __syncthreads();
    if (tid == 0) {
      float b = m->rf[0];
      int bi = m->ri[0];
      for (int w = 1; w < NW; ++w)
        if (m->rf[w] > b || (m->rf[w] == b && m->ri[w] < bi)) {
          b = m->rf[w];
          bi = m->ri[w];
        }
      m->ri[0] = bi;
      m->rf[0] = b;
    }
    if constexpr (DRAW == DRAW_SHARD_RACE) {
      // this slice's best p / E, its global id and logit; the finish takes the best slice
      if (tid == 0) {
        const int bi = m->ri[0];
        dsv41_full_pick pk;
        pk.id = -1;
        pk.z = NEG_INF;
        pk.ratio = -1.0f;
        if (bi != 0x7FFFFFFF) {
          const bool pen = p.has_pen && ((h.bitmap[bi >> 5] >> (bi & 31)) & 1u);
          pk.id = (int64_t)bi + p.voff;
          pk.z = pen ? penz[slot_of(h, bi)] : load_one<TIn>(rs, bi) / p.T;
          pk.ratio = m->rf[0];
        }
        p.sh_out_picks[row] = pk;
      }
      return;
    }
    // the log-prob against the exact total, as the other draws report it
    if (tid == 0) {
      const int bi = m->ri[0];
      const int64_t tok = bi == 0x7FFFFFFF ? 0 : bi;
      float ztok = M;
      if (bi != 0x7FFFFFFF) {
        const bool pen = p.has_pen && ((h.bitmap[bi >> 5] >> (bi & 31)) & 1u);
        ztok = pen ? penz[slot_of(h, bi)] : load_one<TIn>(rs, bi) / p.T;
      }
      write_result(p, row, m, tok, row_lp(ztok, S), p.V);
    }
    return;
  }

  if constexpr (DRAW == DRAW_SHARD_MASS) {
    // this slice's exact mass against the gathered maximum; the draw step gathers them
    if (tid == 0) p.sh_out_masses[row] = S;
    return;
  }
  // first chunk whose maximum is the row maximum, first history token at it (greedy; a
  // uniform condition, so the block reductions inside are reached by every thread or none)
  int cfirst = NC, pfirst = 0x7FFFFFFF;
  if (!PLACES || p.greedy) {
    for (int c = tid; c < NC; c += NT)
      if (span_max(c) == M) cfirst = min(cfirst, c);
    for (int s = tid; s < U; s += NT)
      if (penz[s] == M) pfirst = min(pfirst, (int)h.tok[s]);
    cfirst = block_min_i<NT>(cfirst, m);
    pfirst = block_min_i<NT>(pfirst, m);
  }

  if (wid == 0) {
    int64_t tok = 0;
    float ztok = M;
    // one chunk re-read: z of its elements, history tokens restored from penz
    auto chunk_z = [&](int c, float(&z)[G]) {
      const int base = c * 64 * G + lane * G;
      Raw<TIn, G> r;
      load_group<TIn, G, VEC, FULL_CPOL>(r, rs, base);
      float x[G];
      unpack(r, x);
      int dummy = 0;
      make_z<G, true>(x, base, p, h.bitmap, z, dummy);
      if (p.has_pen) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const int v = base + j;
          if (v < p.V && ((h.bitmap[v >> 5] >> (v & 31)) & 1u)) z[j] = penz[slot_of(h, v)];
        }
      }
    };
    if (!PLACES || p.greedy) {  // greedy; the state carries the first argmax
      int best = pfirst;
      if (cfirst < NC) {
        float z[G];
        chunk_z(cfirst, z);
        const int base = cfirst * 64 * G + lane * G;
        int first = 0x7FFFFFFF;
#pragma unroll
        for (int j = G - 1; j >= 0; --j)
          if (z[j] == M && base + j < p.V) first = base + j;
        first = wave_min_i(first);
        best = min(best, first);
      }
      tok = best;
      ztok = M;
    } else if (PLACES && m->bi[0] >= 0) {
      // The first id of the target's chunk whose boundary in Q units exceeds what the chunk
      // owes: lanes 0 .. 256/G - 1 hold the chunk's 256 ids.  An id outside the history
      // carries w_i against the chunk maximum, a history id its mass against Mref.
      const int ce = m->bi[0];
      const uint64_t need = m->bu[0];
      const float mc = em[ce];
      const float g = mass_ff(mc, Mref);
      const bool act = lane < MASS_CHUNK / G;
      const int base = ce * MASS_CHUNK + lane * G;
      Raw<TIn, G> r;
      load_group<TIn, G, VEC, FULL_CPOL>(r, rs, base);  // lanes past the chunk: not used
      float x[G], z[G];
      unpack(r, x);
      int dummy = 0;
      make_z<G, true>(x, base, p, h.bitmap, z, dummy);  // history ids and the tail read -inf
      uint64_t wq[G], hq[G];
      uint64_t sw = 0, sh = 0;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const int v = base + j;
        const bool hist = act && p.has_pen && v < p.V && ((h.bitmap[v >> 5] >> (v & 31)) & 1u);
        wq[j] = act ? mass_of(z[j], mc) : 0;
        hq[j] = 0;
        if (hist) {
          z[j] = penz[slot_of(h, v)];
          hq[j] = mass_of(z[j], Mref);
        }
        sw += wq[j];
        sh += hq[j];
      }
      uint64_t cw = wave_incl_scan_u64(sw, lane) - sw, ch = wave_incl_scan_u64(sh, lane) - sh;
      int pick = -1;
      float zp = NEG_INF;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        cw += wq[j];
        ch += hq[j];
        if (act && pick < 0 && need < scale_mass(cw, g) + ch) {
          pick = base + j;
          zp = z[j];
        }
      }
      const unsigned long long hit = __ballot(pick >= 0);
      if (hit) {
        const int src_lane = __ffsll((long long)hit) - 1;
        tok = __shfl(pick, src_lane);
        ztok = __shfl(zp, src_lane);
      }
    }
    // else: no mass at all, only rows without a finite maximum (flagged non-finite)
    if (lane == 0) {
      if constexpr (DRAW == DRAW_STATE) {
        dsv41_full_state st;
        st.max_z = M;
        st.status = m->status;
        st.mass = (double)S * 0x1p-43;
        st.argmax = tok + p.voff;
        st.reserved = 0;
        p.sh_out_states[row] = st;
      } else if constexpr (DRAW == DRAW_SHARD_CDF) {
        // The owning slice's own masses must hold the target; when they do not (masses
        // gathered from other knobs, history or logits than this step's), no id is placed
        // and the finish flags the row.
        p.sh_out_picks[row] = dsv41_full_pick{m->bi[0] >= 0 ? tok + p.voff : -1, ztok, 0.0f};
      } else {
        write_result(p, row, m, tok, MASSES ? row_lp(ztok, S) : __builtin_nanf(""), p.V);
      }
    }
  }
}

// ====================================================================== TOPK
// Wave-uniform values moved to scalar registers (they come from LDS or lane
// reductions, which leave them in vector registers).
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uni(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ uint64_t uni(uint64_t v) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(v >> 32)) << 32) |
         (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
}

// The k-th largest of n unique u64 keys in LDS (1 <= k <= n): eight passes of an 8-bit
// radix selection with u32 bin counts in cnt[256].
template <int NT, bool SHORT = false>
__device__ __forceinline__ uint64_t kth_largest(const uint64_t* keys, int n, int k, uint32_t* cnt, Misc* m) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  uint64_t prefix = 0, mask = 0;
  uint32_t target = (uint32_t)k;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += NT) cnt[i] = 0;
    __syncthreads();
    for (int i = tid; i < n; i += NT) {
      const uint64_t key = keys[i];
      if ((key & mask) == prefix) atomicAdd(&cnt[(key >> shift) & 255], 1u);
    }
    __syncthreads();
    if (wid == 0) {
      // bins in descending digit order: lane l holds digits 255-4l .. 252-4l
      uint32_t c[4], sum = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        c[q] = cnt[255 - (lane * 4 + q)];
        sum += c[q];
      }
      // (shuffles, not the DPP scan: with DPP here topk_kernel's scalar spills move from
      // vector-register lanes to scratch memory)
      const uint32_t incl = (uint32_t)wave_incl_scan_i((int)sum, lane);
      const uint32_t before = incl - sum;
      if (before < target && target <= incl) {
        uint32_t acc = before;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          if (acc < target && target <= acc + c[q]) {
            m->bi[0] = 255 - (lane * 4 + q);
            m->bi[1] = (int)(target - acc);
            if constexpr (SHORT) m->bi[2] = (int)c[q];
          }
          acc += c[q];
        }
      }
    }
    __syncthreads();
    const int digit = uni(m->bi[0]);
    target = (uint32_t)uni(m->bi[1]);
    const int in_bin = SHORT ? uni(m->bi[2]) : 0;
    __syncthreads();
    prefix |= (uint64_t)digit << shift;
    mask |= (uint64_t)0xFF << shift;
    if constexpr (SHORT) {
      if (in_bin == 1 && shift > 0) {
        // One key left under the prefix (keys are unique): it is the k-th largest.  One
        // scan finds it instead of the remaining digit passes (random keys settle in 2-3
        // bytes).  (Kernels whose occupancy the extra registers would cost keep 8 passes.)
        for (int i = tid; i < n; i += NT)
          if ((keys[i] & mask) == prefix) m->bu[0] = keys[i];
        __syncthreads();
        const uint64_t key = m->bu[0];
        __syncthreads();
        return key;
      }
    }
  }
  return prefix;
}

// Keeps the candidate buffer at its top_k and within the min-p bound of mrun (a lower
// bound of the row maximum); returns the new count and updates tau / tau_key.  The
// top_k-th key comes from a radix selection (8 passes of 8 bits over the unique u64
// keys), and the survivors are compacted in place, in buffer order: about 50x less LDS
// traffic than sorting the buffer.  The buffer is left unsorted.
template <int NT, bool SHORT = false>
__device__ __forceinline__ int topk_compact(uint64_t* cand, int n, Misc* m, const Params& p, float mrun, float& tau,
                                            uint64_t& tau_key, uint64_t* hist) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const bool mp = p.min_p > 0.0f && mrun > NEG_INF;
  int el = n;
  if (mp) {
    int e = 0;
    for (int i = tid; i < n; i += NT) e += minp_ok(ckey_z(cand[i]), mrun, p) ? 1 : 0;
    el = block_sum_i<NT>(e, m);
  }
  el = uni(el);
  // With at least top_k keys inside the min-p bound the top_k largest keys survive (they
  // pass it: the bound keeps a prefix of the key order); otherwise exactly those inside.
  const bool by_key = el >= p.top_k && p.top_k > 0;
  uint64_t thr = 0;
  if (by_key) {
    // Under the internal bound, el == top_k keys inside the bound all survive, which is
    // the min-p compaction itself; only more than top_k of them send the row to the
    // fallback (as in block_final).
    if (p.topk_internal && el > p.top_k && tid == 0) atomicOr(&m->status, ST_FALLBACK);
    thr = uni(kth_largest<NT, SHORT>(cand, n, p.top_k, reinterpret_cast<uint32_t*>(hist), m));
    tau_key = thr;
    tau = ckey_z(thr);
  }
  // In place, NT keys a round: a round reads its window [r0, r0 + NT), and its writes
  // land below r0 + NT (at most r0 keys survive the earlier rounds), after every read of
  // the window and before any read of the next one.
  int total = 0;
  for (int r0 = 0; r0 < n; r0 += NT) {
    const int i = r0 + tid;
    const uint64_t k = i < n ? cand[i] : 0;
    const bool ok = i < n && (by_key ? k >= thr : (!mp || minp_ok(ckey_z(k), mrun, p)));
    const unsigned long long bal = __ballot(ok);
    if (lane == 0) m->ri[wid] = (int)__popcll(bal);
    __syncthreads();
    int before = 0, round = 0;
    for (int w = 0; w < NT / 64; ++w) {
      const int t = uni(m->ri[w]);
      if (w < wid) before += t;
      round += t;
    }
    if (ok) cand[total + before + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u))] = k;
    total += round;
    __syncthreads();
  }
  return uni(total);
}

// Lane exchange of a u64 with lane ^ j, all 64 lanes active.  j = 1, 2 and 8 are one
// DPP move per half (quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_ror:8); j = 4 takes
// row_ror:4 or row_ror:12, whichever brings lane ^ 4 (ror4 says so per lane); larger j
// cross 16-lane rows and go through the LDS crossbar.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, true);  // in-row sources: no old value
}
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  return ((uint64_t)dpp_u32<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_u32<CTRL>((uint32_t)v);
}
__device__ __forceinline__ uint64_t lane_xor_u64(uint64_t v, int j, bool ror4) {
  switch (j) {
    case 1:
      return dpp_u64<0xB1>(v);
    case 2:
      return dpp_u64<0x4E>(v);
    case 4: {
      const uint64_t a = dpp_u64<0x124>(v), b = dpp_u64<0x12C>(v);
      return ror4 ? a : b;
    }
    case 8:
      return dpp_u64<0x128>(v);
    default:
      return __shfl_xor(v, j);
  }
}

// Descending sort of 64*R u64 keys held by one wave, key at position r*64 + lane in
// k[r], by the bitonic network (stride >= 64: within the lane; below: lane exchange).
template <int R>
__device__ __forceinline__ void wave_sort_desc(uint64_t (&k)[R], int lane) {
  constexpr int N = 64 * R;
  const bool ror4 = dpp_u32<0x124>((uint32_t)lane) == (uint32_t)(lane ^ 4);
#pragma unroll
  for (int s = 2; s <= N; s <<= 1) {
#pragma unroll
    for (int j = s >> 1; j > 0; j >>= 1) {
      if (j >= 64) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int pr = r ^ (j >> 6);
          if (pr > r) {
            const bool desc = ((r * 64) & s) == 0;  // block direction (s >= 128: lane bits do not matter)
            const uint64_t a = k[r], b = k[pr];
            const bool sw = desc ? (a < b) : (a > b);
            k[r] = sw ? b : a;
            k[pr] = sw ? a : b;
          }
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const uint64_t o = lane_xor_u64(k[r], j, ror4);
          const bool desc = ((r * 64 + lane) & s) == 0;
          const bool lower = (lane & j) == 0;
          const bool take_max = lower == desc;
          k[r] = take_max ? (k[r] > o ? k[r] : o) : (k[r] < o ? k[r] : o);
        }
      }
    }
  }
}

// Top 64 of two descending 64-key sequences, one key per lane: v holds one sequence and
// b the other reversed over the lanes (b at lane i is its key 63 - i).  max(v, b) is then a
// bitonic sequence holding the 64 largest keys, which the bitonic merge network sorts
// descending again.
__device__ __forceinline__ uint64_t wave_merge_top64(uint64_t v, uint64_t b, int lane) {
  v = v > b ? v : b;
  const bool ror4 = dpp_u32<0x124>((uint32_t)lane) == (uint32_t)(lane ^ 4);
#pragma unroll
  for (int j = 32; j > 0; j >>= 1) {
    const uint64_t o = lane_xor_u64(v, j, ror4);
    const bool lower = (lane & j) == 0;
    v = lower ? (v > o ? v : o) : (v < o ? v : o);
  }
  return v;
}

// A lower bound of a top_k threshold from one batch of a wave (top_k <= 64 * R): each lane
// offers its R largest finite logits among the batch's in-range non-history elements; if the
// wave offers at least top_k of them, tau becomes one float below RN(x_k / T), x_k the
// top_k-th largest offer.  Those top_k offers are distinct elements with z >= RN(x_k / T)
// (RN(x / T) is non-decreasing in x), so no element at or below tau ranks in the top_k.
template <int R, int NT, int PFN, int G>
__device__ __forceinline__ void seed_tau(const float (&x)[PFN][G], int t0, const Hist& h, const Params& p,
                                         float& tau) {
  const int lane = threadIdx.x & 63;
  float top[R];
#pragma unroll
  for (int r = 0; r < R; ++r) top[r] = NEG_INF;
#pragma unroll
  for (int k = 0; k < PFN; ++k) {
    const int base = (t0 + k) * NT * G + (int)threadIdx.x * G;
    const uint32_t pen = p.has_pen && base < p.V ? (h.bitmap[base >> 5] >> (base & 31)) & ((1u << G) - 1u) : 0u;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const float v = x[k][j];
      if (base + j < p.V && !((pen >> j) & 1u) && isfinite(v)) {
        if constexpr (R == 1) {
          top[0] = fmaxf(top[0], v);
        } else {
#pragma unroll
          for (int r = R - 1; r > 0; --r) top[r] = v > top[r - 1] ? top[r - 1] : fmaxf(top[r], v);
          top[0] = fmaxf(top[0], v);
        }
      }
    }
  }
  uint64_t key[R];
#pragma unroll
  for (int r = 0; r < R; ++r)
    key[r] = top[r] > NEG_INF ? ((uint64_t)okey(top[r]) << 32) | (uint32_t)(r * 64 + lane) : 0;
  wave_sort_desc<R>(key, lane);
  const int pos = p.top_k - 1;
  uint64_t sel = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r == (pos >> 6)) sel = key[r];
  const uint64_t kth = __shfl(sel, pos & 63);
  if (kth != 0) tau = next_down(div_T(okey_inv((uint32_t)(kth >> 32)), p));
}

// Inclusive prefix of x over positions r*64 + lane; returns the total.
template <int R>
__device__ __forceinline__ uint64_t wave_prefix(const uint64_t (&x)[R], uint64_t (&incl)[R], int lane) {
  uint64_t carry = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    incl[r] = wave_incl_scan_u64(x[r], lane) + carry;
    carry = __shfl(incl[r], 63);
  }
  return carry;
}

// Descending order of n <= 64 unique keys, one per lane (lanes >= n hold 0, below every
// key), by rank: each lane counts the keys in buf[0, n) above its own and places its key
// there; buf then holds the sorted keys and each lane reads back its position.  The
// result is the bitonic network's, in about 2n LDS broadcast reads instead of 21
// exchange steps (the final selections of typical rows hold a few keys).
__device__ __forceinline__ uint64_t wave_rank_desc(uint64_t v, uint64_t* buf, int n, int lane) {
  int rank = 0;
  for (int i = 0; i < n; ++i) rank += buf[i] > v ? 1 : 0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (lane < n) buf[rank] = v;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  return lane < n ? buf[lane] : 0;
}

// Final selection of the TOPK kernel by one wave when 1 <= n <= 64*R candidates: the
// same decisions as the workgroup path (min-p, top-k, top-p over exact integer masses,
// inverse-CDF draw in vocabulary order), with every step in registers.  cand (LDS, this
// wave's to overwrite) holds the keys; with R = 1 the two sorts go by rank through it.
// DPP: the kept set's fp64 exp sum by the DPP scan (select_kernel and merge_kernel; the
// in-place copy in topk_kernel keeps the shuffle sum, which leaves that kernel's code as it is)
template <int R, bool DPP = false>
__device__ __forceinline__ void wave_final(const Params& p, int row, Misc* m, uint64_t* cand, int n, float u) {
  const int lane = threadIdx.x & 63;
  uint64_t k[R];
#pragma unroll
  for (int r = 0; r < R; ++r) k[r] = r * 64 + lane < n ? cand[r * 64 + lane] : 0;  // 0 is below every key
  if constexpr (R == 1) k[0] = wave_rank_desc(k[0], cand, n, lane);
  else wave_sort_desc<R>(k, lane);
  const uint64_t k0 = __shfl(k[0], 0);
  const float zmax = ckey_z(k0);
  int el = 0;
#pragma unroll
  for (int r = 0; r < R; ++r)
    el += (int)__popcll(__ballot(r * 64 + lane < n && minp_ok(ckey_z(k[r]), zmax, p)));
  const int K = min(p.top_k, el);
  uint64_t q[R], pre[R];
#pragma unroll
  for (int r = 0; r < R; ++r) q[r] = r * 64 + lane < K ? mass_of(ckey_z(k[r]), zmax) : 0;
  const uint64_t SK = wave_prefix<R>(q, pre, lane);
  int n_keep = K;
  uint64_t S = SK;
  if (p.top_p < 1.0f) {
    const uint64_t thr = top_p_threshold(p.top_p, SK);
    int first = -1;
#pragma unroll
    for (int r = R - 1; r >= 0; --r) {
      const unsigned long long b = __ballot(r * 64 + lane < K && pre[r] >= thr);
      if (b) {
        first = r * 64 + (int)__builtin_ctzll(b);
        S = __shfl(pre[r], first & 63);
      }
    }
    if (first < 0) {  // unreachable: the total reaches every threshold
      first = K - 1;
      S = SK;
    }
    n_keep = first + 1;
  }
  double es = 0.0;
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (r * 64 + lane < n_keep) es += exp_det((double)ckey_z(k[r]) - (double)zmax);
  const double esum = DPP ? wave_total_d(es) : wave_sum_d(es);
  int64_t tok = (int64_t)ckey_idx(k0);
  float ztok = zmax;
  if (!p.greedy) {
    // kept candidates in vocabulary order: ~(index, z) sorts descending as index ascending
    uint64_t k2[R];
#pragma unroll
    for (int r = 0; r < R; ++r)
      k2[r] = r * 64 + lane < n_keep ? ~(((uint64_t)ckey_idx(k[r]) << 32) | (k[r] >> 32)) : 0;
    if constexpr (R == 1) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      cand[lane] = k2[0];  // (the sorted keys stay in k)
      k2[0] = wave_rank_desc(k2[0], cand, n_keep, lane);
    } else {
      wave_sort_desc<R>(k2, lane);
    }
    const uint64_t t = draw_target(u, S);
    uint64_t w[R], cum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) w[r] = r * 64 + lane < n_keep ? mass_of(okey_inv((uint32_t)~k2[r]), zmax) : 0;
    wave_prefix<R>(w, cum, lane);
    bool done = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const unsigned long long b = __ballot(r * 64 + lane < n_keep && cum[r] > t);
      if (b && !done) {
        const uint64_t key = ~__shfl(k2[r], (int)__builtin_ctzll(b));
        tok = (int64_t)(key >> 32);
        ztok = okey_inv((uint32_t)key);
        done = true;
      }
    }
  }
  if (lane == 0) {
    const float lp = (float)(((double)ztok - (double)zmax) - log(esum));
    write_result(p, row, m, tok, lp, n_keep);
  }
}

// Final selection over the n candidate keys in cand by the whole workgroup: bitonic sort,
// then exact scans for min-p, top-k and top-p, and the draw by radix selection.  cand
// holds max(n, 2 * min(top_k, n)) keys (the masses reuse the space past the top-k);
// hist is 256 keys of scratch.
template <int NT>
__device__ __forceinline__ void block_final(const Params& p, int row, Misc* m, uint64_t* cand, int n,
                                            uint64_t* hist) {
  const int tid = threadIdx.x;
  bitonic_sort_desc<NT>(cand, n);
  const float u = row_uniform(p, row, m);
  if (n == 0) {  // only possible for rows without a finite maximum
    __syncthreads();
    if (tid == 0) {
      m->status |= ST_NONFINITE;
      write_result(p, row, m, -1, 0.0f, 0);
    }
    return;
  }
  const float zmax = ckey_z(cand[0]);
  int el = 0;
  for (int i = tid; i < n; i += NT) el += minp_ok(ckey_z(cand[i]), zmax, p) ? 1 : 0;
  el = block_sum_i<NT>(el, m);
  if (p.topk_internal && el > p.top_k && tid == 0) atomicOr(&m->status, ST_FALLBACK);
  const int K = min(p.top_k, el);
  uint64_t* q = cand + K;  // the keys past the top-k are not needed again
  for (int i = tid; i < K; i += NT) q[i] = mass_of(ckey_z(cand[i]), zmax);
  __syncthreads();
  int n_keep = K;
  uint64_t S;
  if (p.top_p < 1.0f) {
    block_incl_scan_u64<NT>(q, K, m);
    const uint64_t thr = top_p_threshold(p.top_p, q[K - 1]);
    if (tid == 0) m->bi[1] = K - 1;
    __syncthreads();
    for (int i = tid; i < K; i += NT)
      if (q[i] >= thr && (i == 0 || q[i - 1] < thr)) m->bi[1] = i;
    __syncthreads();
    n_keep = m->bi[1] + 1;
    S = q[n_keep - 1];
    __syncthreads();
  } else {
    uint64_t s = 0;
    for (int i = tid; i < K; i += NT) s += q[i];
    S = block_sum_u64<NT>(s, m);
  }
  double es = 0.0;
  for (int i = tid; i < n_keep; i += NT) es += exp_det((double)ckey_z(cand[i]) - (double)zmax);
  const double esum = block_sum_d<NT>(es, m);

  int64_t tok;
  float ztok;
  if (p.greedy) {
    tok = ckey_idx(cand[0]);
    ztok = zmax;
  } else {
    const uint64_t t = draw_target(u, S);
    bool found = false;
    const uint64_t idx = radix_select<NT, false, 24>(
        [&](auto&& f) {
          for (int i = tid; i < n_keep; i += NT) {
            const uint64_t k = cand[i];
            f((uint64_t)ckey_idx(k), mass_of(ckey_z(k), zmax));
          }
        },
        t + 1, hist, m, &found);
    tok = found ? (int64_t)idx : (int64_t)ckey_idx(cand[0]);
    if (tid == 0) m->bf[0] = zmax;
    __syncthreads();
    for (int i = tid; i < n_keep; i += NT)
      if (ckey_idx(cand[i]) == (uint32_t)tok) m->bf[0] = ckey_z(cand[i]);
    __syncthreads();
    ztok = m->bf[0];
  }
  if (tid == 0) {
    const float lp = (float)(((double)ztok - (double)zmax) - log(esum));
    write_result(p, row, m, tok, lp, n_keep);
  }
}

// EMIT: the launch covers one vocabulary shard; each row's candidates leave for
// merge_kernel instead of being sampled here.
// NTK = 256 (deferred batches whose tables fit four workgroups per CU) holds 16 history ids
// per thread as int32: 4096 ids in the registers that 8 int64 ids take at NTK = 512.
//
// SLICED (with EMIT): a batch too small to fill the GPU, spread over it.  Each workgroup
// emits its slice's exact local top_k, as a vocabulary shard does, into
// [n_slices, nrows, emit_cap]; merge_kernel then finishes every row exactly.
// GATHER = false: a batch that gathers no history slots (no penalties, or lowering ones,
// which the stream applies itself), whose batch loop then holds no gathered-slot code:
// fewer live registers on every batch.
// SEED (256-thread row launches of top_k <= 256 without min-p): the first batch's threshold
// is the largest of the waves' top_k-th largest offers, four per lane, over one barrier.
template <typename TIn, bool VEC, bool EMIT = false, int NTK = TOPK_NT, bool SLICED = false, bool GATHER = true,
          bool SEED = false>
__global__ __launch_bounds__(NTK) void topk_kernel(Params p) {
  static_assert(!SLICED || EMIT, "a sliced launch emits candidate lists");
  const int row = SLICED ? (int)blockIdx.x / p.n_slices : (int)blockIdx.x;
  const int erow = SLICED ? ((int)blockIdx.x % p.n_slices) * p.nrows + row : row;  // output slot
  if constexpr (SLICED) {
    const int v0 = ((int)blockIdx.x % p.n_slices) * p.slice_w;
    p.voff = v0;
    p.V = min(p.slice_w, p.vfull - v0);
    p.logits = reinterpret_cast<const TIn*>(p.logits) + v0;
  }
  constexpr int NT = NTK, NW = NT / 64, G = TOPK_G, TILE = NT * G, HR = 4096 / NT;
  // the radix selection's early exit where its registers cost no occupancy
  constexpr bool SHORT_SEL = NT < TOPK_NT || (EMIT && VEC && sizeof(TIn) == 4);
  using IdT = std::conditional_t<(NT < TOPK_NT), int32_t, int64_t>;
  constexpr int NE = PF * G + 1;  // elements per thread in one batch round (+1 history slot)
  extern __shared__ __align__(16) unsigned char smem[];
  const Layout L = make_layout<MODE_TOPK, G>(p.V, p.words, p.ucap, p.cap, p.no_ranks == 0);
  Misc* m = reinterpret_cast<Misc*>(smem + L.misc);
  const Hist h = hist_tables(smem, L);
  uint64_t* hist = reinterpret_cast<uint64_t*>(smem + L.hist256);
  uint64_t* cand = reinterpret_cast<uint64_t*>(smem + L.mode0);

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  HistIds<HR, IdT> hi;
  load_history<NT, HR>(p, row, hi);
  const TIn* src = row_ptr<TIn>(p, row);
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(src, (uint32_t)p.V * (uint32_t)sizeof(TIn));
  int bad = 0;
  int count = 0;            // candidates stored (uniform across the workgroup)
  float tau = NEG_INF;      // z of the top_k-th candidate once the buffer held top_k
  uint64_t tau_key = 0;
  float wm = NEG_INF;       // this wave's running maximum (a lower bound of the row max)
  float mblk = NEG_INF;     // all waves' running maxima at the last exchange
  int par = 0;
  float ax = 0.0f;             // largest |x| seen by this lane
  float c_tau = __builtin_nanf(""), c_bnd = __builtin_nanf(""), c_thr = NEG_INF;  // x-threshold cache

  // One exchange of per-wave insert counts and running maxima over one barrier; the
  // buffer is compacted when the round could overflow it.  Returns this wave's first
  // position, or -1 when the round does not fit even after compaction.
  auto exchange = [&](uint32_t wn, int& total) -> int {
    if (lane == 0) {
      m->wcnt[par][wid] = (int)wn;
      m->wmax[par][wid] = wm;
    }
    __syncthreads();
    total = 0;
    int before = 0;
    float mb = NEG_INF;
    for (int i = 0; i < NW; ++i) {
      const int v = m->wcnt[par][i];
      total += v;
      if (i < wid) before += v;
      mb = fmaxf(mb, m->wmax[par][i]);
    }
    mblk = uni(mb);
    total = uni(total);
    before = uni(before);
    par ^= 1;
    if (count + total > p.cap) count = topk_compact<NT, SHORT_SEL>(cand, count, m, p, mblk, tau, tau_key, hist);
    return count + total <= p.cap ? count + before : -1;
  };
  // One insertion round of up to M (<= G) elements per thread; always fits, because
  // after a compaction count <= top_k and cap = top_k + TILE.
  auto round = [&](auto&& elem, int M) {
    unsigned long long bal[G];
    uint32_t wn = 0;
#pragma unroll
    for (int j = 0; j < G; ++j) {
      bal[j] = 0;
      if (j < M) {
        uint64_t key;
        bal[j] = __ballot(elem(j, key));
        wn += (uint32_t)__popcll(bal[j]);
      }
    }
    int total;
    int pos = exchange(wn, total);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if (j < M && bal[j]) {
        if ((bal[j] >> lane) & 1ull) {
          uint64_t key;
          elem(j, key);
          cand[pos + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal[j] >> 32),
                                                    __builtin_amdgcn_mbcnt_lo((uint32_t)bal[j], 0u))] = key;
        }
        pos += (int)__popcll(bal[j]);
      }
    }
    count += total;
  };

  int U = 0;
  stream_row<TIn, G, NT, VEC, true>(  // lowering penalties: history tokens are met in the stream
      p, rs, h,
      [&]() {
        if (tid == 0) m->status = 0;
        __syncthreads();
        // with lowering penalties the stream evaluates history tokens itself and needs
        // their counts only for a frequency penalty
        if (p.has_pen) U = build_history<NT, HR, EMIT>(p, row, hi, h, m, !p.pen_lowers || p.pen_counts);
        landed(hi);  // the ids are read under conditions; end their loads on every path
        return U;
      },
      [&](int t0, int nt, Raw<TIn, G>(&R)[PF], int s0, int n_gathered, float gx) {
        const int n = GATHER ? n_gathered : 0;
        // Tiles past the row are read and masked, not skipped, so that every load is
        // consumed (as in full_kernel).
        float x[PF][G];
#pragma unroll
        for (int k = 0; k < PF; ++k) unpack(R[k], x[k]);
        // the batch's first NT history slots, penalized exactly
        float zg = NEG_INF;
        uint32_t tg = 0;
        if (tid < n) {
          const int s = s0 + tid;
          tg = h.tok[s];
          zg = pen_z(gx, count_of(h, s), p);
          if (!isfinite(zg)) bad = 1;
        } else {
          landed(gx);
        }
        float zmx = zg;
        // A wave without a running maximum takes one from this batch's non-history
        // logits before filtering, so that min-p already thins its first batch.
        if (p.min_p > 0.0f && !(fmaxf(wm, mblk) > NEG_INF)) {
          float lx = NEG_INF;
#pragma unroll
          for (int k = 0; k < PF; ++k) {
            const int base = (t0 + k) * TILE + tid * G;
            const uint32_t pen = p.has_pen && base < p.V ? (h.bitmap[base >> 5] >> (base & 31)) & ((1u << G) - 1u) : 0u;
#pragma unroll
            for (int j = 0; j < G; ++j)
              if (base + j < p.V && !((pen >> j) & 1u)) lx = fmaxf(lx, x[k][j]);
          }
          // RN(x/T) is non-decreasing in x: the largest z is the quotient of the largest x
          if (lx > NEG_INF) zmx = fmaxf(zmx, lx / p.T);
        }
        // A wave without a top_k threshold (top_k <= 64) takes one before filtering its
        // first batch: each lane offers its largest finite non-history logit, so the
        // top_k-th largest offer belongs to top_k distinct elements and the top_k-th
        // largest z of the row (or shard) is at least its quotient.  tau one float below
        // that quotient admits every element that can rank in the top_k (tau_key stays 0:
        // keys then compare only against tau's float).  Without it the first batch fills
        // the buffer and compacts it several times before any threshold exists.
        // (256-thread and shard or slice launches: the 512-thread row kernel has no register
        // left for it at two workgroups per CU)
        // SEED takes four offers a lane, so each wave's bound is near its own top_k-th largest
        // logit, and the largest of the waves' bounds (each at most the row's top_k-th
        // largest z) lets about top_k elements of the batch through instead of every
        // wave's share.  The condition is uniform over the workgroup (tau is, once set).
        if constexpr (SEED) {
          if (p.top_k >= 1 && p.top_k <= 4 * 64 && !(tau > NEG_INF)) {
            float tw = NEG_INF;
            seed_tau<4, NT>(x, t0, h, p, tw);
            if (lane == 0) m->rf[wid] = tw;
            __syncthreads();
            float tb = NEG_INF;
#pragma unroll
            for (int i = 0; i < NW; ++i) tb = fmaxf(tb, m->rf[i]);
            tau = uni(tb);
          }
        } else if constexpr (EMIT || NT < TOPK_NT) {
          if (p.top_k >= 1 && p.top_k <= 64 && !(tau > NEG_INF)) seed_tau<1, NT>(x, t0, h, p, tau);
        }
        // (skipped when no lane holds a finite value: the maximum is then unchanged; the
        // test costs the unaligned-row instantiations their fourth wave per SIMD)
        // (SEED launches have no min-p, the one use of the running maximum: they keep none)
        if constexpr (!SEED) {
          if (!VEC || __ballot(zmx > NEG_INF)) wm = uni(fmaxf(wm, wave_max_dpp(zmx)));
        }
        const float bnd = minp_bound_f(fmaxf(wm, mblk), p.lmin_f);
        if (!(tau == c_tau && bnd == c_bnd)) {
          c_tau = tau;
          c_bnd = bnd;
          c_thr = uni(x_threshold(tau, bnd, p));
        }
        const float th = c_thr;
        const uint64_t tk = tau_key;
        // Stream elements: one compare per logit against the raw threshold; the test
        // !(x < th) also passes NaN.  Later tiles hold larger indices, so z > tau
        // suffices against the k-th key; history tokens compare full keys.  |x| is
        // tracked for infinities and for x / T overflow, checked after the stream.
        unsigned long long bal[NE];
        unsigned long long any = 0;
#pragma unroll
        for (int k = 0; k < PF; ++k)
#pragma unroll
          for (int j = 0; j < G; ++j) {
            ax = fmaxf(ax, fabsf(x[k][j]));
            bal[k * G + j] = __ballot(!(x[k][j] < th));
            any |= bal[k * G + j];
          }
        uint32_t wn = 0;  // the wave's passers, counted where they are decided
        if (any) {
          // Passers are rare once the thresholds settle.  Positions past the row drop
          // out and a non-finite logit flags the row.  The passers' z replaces x in
          // place.  A history token under lowering penalties has z = pen_z(x) <= x / T,
          // so it can only qualify when x passes: its exact z takes the full test here.
          // Otherwise history tokens drop out and the gather brings their exact values.
          // Every element above the running maximum passes, so the passers' largest z
          // keeps that maximum exact.
          float pz = NEG_INF;
          // this lane's history bits of each tile, read together up front (the G
          // elements of a lane share one bitmap word)
          uint32_t hb[PF];
#pragma unroll
          for (int k = 0; k < PF; ++k) {
            const int base = (t0 + k) * TILE + tid * G;
            hb[k] = p.has_pen && base < p.V ? (h.bitmap[base >> 5] >> (base & 31)) & ((1u << G) - 1u) : 0u;
          }
#pragma unroll
          for (int k = 0; k < PF; ++k) {
            const int base = (t0 + k) * TILE + tid * G;
#pragma unroll
            for (int j = 0; j < G; ++j) {
              const int e = k * G + j;
              if (bal[e]) {
                bool ok = (bal[e] >> lane) & 1ull;
                if (ok) {
                  const int idx = base + j;
                  const float xv = x[k][j];
                  const bool in = idx < p.V;
                  if (in && !isfinite(xv)) bad = 1;
                  ok = in && isfinite(xv);
                  if (ok) {
                    if ((hb[k] >> j) & 1u) {
                      if (p.pen_lowers) {
                        const float z = pen_z(xv, p.pen_counts ? count_of(h, slot_of(h, idx)) : 1u, p);
                        if (!isfinite(z)) bad = 1;
                        ok = isfinite(z) && z > tau && z >= bnd;
                        if (isfinite(z)) pz = fmaxf(pz, z);
                        x[k][j] = z;
                      } else {
                        ok = false;
                      }
                    } else {
                      const float z = div_T(xv, p);
                      pz = fmaxf(pz, z);
                      x[k][j] = z;
                    }
                  }
                }
                bal[e] = __ballot(ok);
                wn += (uint32_t)__popcll(bal[e]);
              }
            }
          }
          if constexpr (!SEED) wm = uni(fmaxf(wm, wave_max_dpp(pz)));
        }
        // the batch's gathered history slot (none when the batch gathered none: zg = -inf)
        uint64_t kg = 0;
        bal[NE - 1] = 0;
        if (n > 0) {
          kg = ckey(zg, tg);
          bal[NE - 1] = __ballot(zg > NEG_INF && kg > tk && zg >= bnd);
          wn += (uint32_t)__popcll(bal[NE - 1]);
        }
        int total;
        int pos = exchange(wn, total);
        if (pos >= 0) {
          auto insert = [&](int e, uint64_t b) {
            if ((b >> lane) & 1ull) {
              const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
              const uint64_t key =
                  e == NE - 1 ? kg : ckey(x[e / G][e % G], (uint32_t)((t0 + e / G) * TILE + tid * G + e % G));
              cand[pos + below] = key;
            }
            pos += (int)__popcll(b);
          };
          // the stream elements' ballots are all zero when nothing passed: the common
          // batch then reads none of them back
          if (any) {
#pragma unroll
            for (int e = 0; e < NE - 1; ++e)
              if (bal[e]) insert(e, bal[e]);
          }
          if (bal[NE - 1]) insert(NE - 1, bal[NE - 1]);
          count += total;
        } else {
          // the batch does not fit: one round per tile, then the history round; each
          // round tests the passers' z against the compacted buffer's tau
#pragma unroll
          for (int k = 0; k < PF; ++k) {
            const float tau2 = tau;
            const int base = (t0 + k) * TILE + tid * G;
            round([&](int j, uint64_t& key) {
                    key = ckey(x[k][j], (uint32_t)(base + j));
                    return ((bal[k * G + j] >> lane) & 1ull) && x[k][j] > tau2 && x[k][j] >= bnd;
                  }, G);
          }
          const uint64_t tk2 = tau_key;
          round([&](int, uint64_t& key) {
                  key = kg;
                  return zg > NEG_INF && kg > tk2 && zg >= bnd;
                }, 1);
        }
        // history slots past the first NT of this batch
        for (int i0 = NT; i0 < n; i0 += NT) {
          const int i = i0 + tid;
          float z2 = NEG_INF;
          uint32_t t2 = 0;
          if (i < n) {
            const int s = s0 + i;
            t2 = h.tok[s];
            z2 = pen_z(load_one<TIn>(rs, (int)t2), count_of(h, s), p);
            if (!isfinite(z2)) bad = 1;
          }
          if constexpr (!SEED) wm = uni(fmaxf(wm, wave_max_dpp(z2)));
          const float bnd2 = minp_bound_f(fmaxf(wm, mblk), p.lmin_f);
          const uint64_t k2 = ckey(z2, t2), tk3 = tau_key;
          round([&](int, uint64_t& key) {
                  key = k2;
                  return z2 > NEG_INF && k2 > tk3 && z2 >= bnd2;
                }, 1);
        }
        // A buffer well above its top_k compacts before the next batch instead of when full:
        // the threshold then rises to the top_k-th of the elements seen so far, and the
        // batches after pass a few elements each instead of a few percent (measured with
        // top-k 50 alone: 0.886 -> 0.745 ms at E's shape, 32 sliced rows 76.5 -> 50.1 us;
        // the trigger 2 top_k + 128 beat top_k + 192, 4 top_k + 256 and 8 top_k + 256).
        if (count > p.mid_trigger && t0 + PF < nt)
          count = topk_compact<NT, SHORT_SEL>(cand, count, m, p, mblk, tau, tau_key, hist);
      });
  // NaN and +inf logits passed the filter and flagged the row there; -inf, and a finite
  // x whose x / T or penalized value could overflow, show in |x|: rare, so such rows
  // re-check every element
  const float axw = wave_max_dpp(ax);
  const float pen_mag = p.has_pen ? axw * fmaxf(1.0f, p.rp) + fabsf(p.pres) + fabsf(p.freq) * (float)p.hstride : 0.0f;
  if (!isfinite(axw / p.T) || !isfinite(pen_mag / p.T)) atomicOr(&m->status, ST_RECHECK);
  __syncthreads();
  if (m->status & ST_RECHECK) {
    for (int i = tid; i < p.V; i += NT) {
      const bool pen = p.has_pen && ((h.bitmap[i >> 5] >> (i & 31)) & 1u);
      const float xi = load_one<TIn>(rs, i);
      const float z = pen ? pen_z(xi, U > 0 ? count_of(h, slot_of(h, i)) : 1u, p) : xi / p.T;
      if (!isfinite(z)) bad = 1;
    }
    __syncthreads();
    if (tid == 0) m->status &= ~ST_RECHECK;
  }
  if (bad) atomicOr(&m->status, ST_NONFINITE);
  __syncthreads();

  if constexpr (EMIT) {
    // Vocabulary shard: the exact local top_k under the local min-p bound.  The local
    // maximum is at most the row's, so every token of the row's kept set is in its
    // shard's list, and merge_kernel finishes the row from the union of the lists.
    int keep = 0;
    if (count > 0) {
      bitonic_sort_desc<NT>(cand, count);
      const float zmax = ckey_z(cand[0]);
      int el = 0;
      for (int i = tid; i < count; i += NT) el += minp_ok(ckey_z(cand[i]), zmax, p) ? 1 : 0;
      keep = min(p.top_k, block_sum_i<NT>(el, m));
    }
    uint64_t* out = p.emit_keys + (int64_t)erow * p.emit_cap;
    for (int i = tid; i < keep; i += NT) {
      const uint64_t k = cand[i];
      out[i] = ckey(ckey_z(k), ckey_idx(k) + (uint32_t)p.voff);
    }
    if (tid == 0) {
      p.emit_count[erow] = keep;
      p.out_status[erow] = m->status;
    }
    return;
  }

  // The buffer can end above what one wave selects from: without a min-p bound (top-k 50
  // alone ends near 300 keys), or with one taken from a running maximum that rose late.  The
  // final selection keeps a subset of the top_k keys within the min-p bound of the row
  // maximum, so compacting to those changes only the count, which then fits the one-wave
  // selection (deferred, or in place) instead of the block sort.
  int n = count;
  if (n > DEFER_KEYS && ((p.top_k > 0 && p.top_k <= DEFER_KEYS) || p.min_p > 0.0f) && !(m->status & ST_NONFINITE)) {
    float zm = NEG_INF;
    for (int i = tid; i < n; i += NT) zm = fmaxf(zm, ckey_z(cand[i]));
    zm = block_max<NT>(zm, m);
    n = topk_compact<NT, SHORT_SEL>(cand, n, m, p, zm, tau, tau_key, hist);
  }
  // final selection over the candidates: one wave when they fit its registers
  if (p.defer && n >= 1 && n <= DEFER_KEYS) {
    // The selection is a serial chain of about 15k cycles in one wave; select_kernel
    // runs it for all rows at once, so this workgroup's slot goes back to streaming.
    uint64_t* dk = p.defer_keys + (int64_t)row * DEFER_KEYS;
    for (int i = tid; i < n; i += NT) dk[i] = cand[i];
    if (tid == 0) {
      p.defer_count[row] = n;
      p.out_status[row] = m->status;
    }
    return;
  }
  if (p.defer && tid == 0) p.defer_count[row] = 0;
  if (n >= 1 && n <= 4 * 64) {
    if (wid == 0) {
      const float u = row_uniform(p, row, m);
      if (n <= 64) wave_final<1>(p, row, m, cand, n, u);
      else if (n <= 128) wave_final<2>(p, row, m, cand, n, u);
      else wave_final<4>(p, row, m, cand, n, u);
    }
    return;
  }
  block_final<NT>(p, row, m, cand, n, hist);
}

// ====================================================================== GENERIC
template <typename TIn, int G, bool VEC>
__global__ __launch_bounds__(GEN_NT) void generic_kernel(Params p) {
  constexpr int NT = GEN_NT, HR = 4;
  extern __shared__ __align__(16) unsigned char smem[];
  const Layout L = make_layout<MODE_GENERIC, G>(p.V, p.words, p.ucap, 0);
  Misc* m = reinterpret_cast<Misc*>(smem + L.misc);
  const Hist h = hist_tables(smem, L);
  uint64_t* hist = reinterpret_cast<uint64_t*>(smem + L.hist256);

  const int tid = threadIdx.x;
  // One row per workgroup.  A fallback launch (only_flagged, after TOPK or TOPP) walks the
  // batch with a grid of at most FALLBACK_GRID workgroups and redoes only the flagged rows,
  // which are few: a row per workgroup would dispatch the whole batch to find them.
  const int nrows = p.only_flagged ? p.nrows : (int)gridDim.x;
  if (p.only_flagged) {
    // this workgroup's rows' statuses in one parallel read; most launches find none flagged
    const int mine = ((nrows - (int)blockIdx.x) + (int)gridDim.x - 1) / (int)gridDim.x;
    bool flagged = mine > NT;  // (more rows than threads: the loop reads the rest itself)
    for (int j = tid; j < mine && j < NT; j += NT)
      flagged |= (p.out_status[blockIdx.x + j * gridDim.x] & ST_FALLBACK) != 0;
    if (block_sum_i<NT>(flagged ? 1 : 0, m) == 0) return;  // (no static LDS: the launch sets the dynamic maximum)
  }
  for (int row = blockIdx.x; row < nrows; row += gridDim.x) {
    if (p.only_flagged && !(p.out_status[row] & ST_FALLBACK)) continue;  // uniform: one row
    HistIds<HR> hi;
    load_history<NT, HR>(p, row, hi);
    const TIn* src = row_ptr<TIn>(p, row);
    const __amdgpu_buffer_rsrc_t rs = row_rsrc(src, (uint32_t)p.V * (uint32_t)sizeof(TIn));
    float* zr = p.zbuf + (int64_t)row * p.V;
    constexpr int TILE = NT * G;
    int bad = 0;
    int U = 0;
    stream_row<TIn, G, NT, VEC, false>(
        p, rs, h,
        [&]() {
          if (tid == 0) m->status = 0;
          __syncthreads();
          if (p.has_pen) U = build_history<NT, HR>(p, row, hi, h, m);
          landed(hi);  // the ids are read under conditions; end their loads on every path
          return U;
        },
        [&](int t0, int nt, Raw<TIn, G>(&R)[PF], int s0, int n, float gx) {
  #pragma unroll
          for (int k = 0; k < PF; ++k) {
            const int t = t0 + k;
            if (t < nt) {
              const int base = t * TILE + tid * G;
              float x[G], z[G];
              unpack(R[k], x);
              make_z<G, true>(x, base, p, h.bitmap, z, bad);
  #pragma unroll
              for (int j = 0; j < G; ++j)
                if (base + j < p.V) zr[base + j] = z[j];
            }
          }
          // the tiles wrote -inf at history tokens: order those stores before the exact ones
          __threadfence_block();
          __syncthreads();
          for (int i = tid; i < n; i += NT) {
            const int s = s0 + i;
            const float x = i == tid ? gx : load_one<TIn>(rs, (int)h.tok[s]);
            const float z = pen_z(x, count_of(h, s), p);
            if (!isfinite(z)) bad = 1;
            zr[h.tok[s]] = z;
          }
        });
    if (bad) atomicOr(&m->status, ST_NONFINITE);
    __threadfence_block();
    __syncthreads();

    const int V = p.V;
    float bm = NEG_INF;
    int bi = 0x7FFFFFFF;
    for (int i = tid; i < V; i += NT) {
      const float z = zr[i];
      if (z > bm) {
        bm = z;
        bi = i;
      }
    }
    const float zmax = block_max<NT>(bm, m);
    int am = block_min_i<NT>(bm == zmax ? bi : 0x7FFFFFFF, m);
    if (am < 0 || am >= V) am = 0;  // no finite maximum: the row is flagged non-finite
    const float u = row_uniform(p, row, m);

    int el = 0;
    for (int i = tid; i < V; i += NT) el += minp_ok(zr[i], zmax, p) ? 1 : 0;
    el = block_sum_i<NT>(el, m);
    const int K = (p.top_k > 0 && p.top_k < el) ? p.top_k : el;
    bool found = false;
    uint64_t B1 = 0;
    if (K < el) {
      B1 = radix_select<NT, true, 64>(
          [&](auto&& f) {
            for (int i = tid; i < V; i += NT) {
              const float z = zr[i];
              if (minp_ok(z, zmax, p)) f(ckey(z, (uint32_t)i), 1ull);
            }
          },
          (uint64_t)K, hist, m, &found);
    }
    uint64_t B = B1;
    if (p.top_p < 1.0f) {
      uint64_t s1 = 0;
      for (int i = tid; i < V; i += NT) {
        const float z = zr[i];
        if (minp_ok(z, zmax, p) && ckey(z, (uint32_t)i) >= B1) s1 += mass_of(z, zmax);
      }
      s1 = block_sum_u64<NT>(s1, m);
      const uint64_t thr = top_p_threshold(p.top_p, s1);
      B = radix_select<NT, true, 64>(
          [&](auto&& f) {
            for (int i = tid; i < V; i += NT) {
              const float z = zr[i];
              const uint64_t k = ckey(z, (uint32_t)i);
              if (minp_ok(z, zmax, p) && k >= B1) f(k, mass_of(z, zmax));
            }
          },
          thr, hist, m, &found);
      if (!found) B = B1;
    }
    int nk = 0;
    uint64_t sk = 0;
    double es = 0.0;
    for (int i = tid; i < V; i += NT) {
      const float z = zr[i];
      if (minp_ok(z, zmax, p) && ckey(z, (uint32_t)i) >= B) {
        ++nk;
        sk += mass_of(z, zmax);
        es += exp_det((double)z - (double)zmax);
      }
    }
    nk = block_sum_i<NT>(nk, m);
    sk = block_sum_u64<NT>(sk, m);
    const double esum = block_sum_d<NT>(es, m);
    int64_t tok = am;
    if (!p.greedy) {
      const uint64_t t = draw_target(u, sk);
      const uint64_t idx = radix_select<NT, false, 24>(
          [&](auto&& f) {
            for (int i = tid; i < V; i += NT) {
              const float z = zr[i];
              if (minp_ok(z, zmax, p) && ckey(z, (uint32_t)i) >= B) f((uint64_t)i, mass_of(z, zmax));
            }
          },
          t + 1, hist, m, &found);
      if (found) tok = (int64_t)idx;
    }
    if (tid == 0) {
      const float ztok = zr[tok];
      const float lp = (float)(((double)ztok - (double)zmax) - log(esum));
      write_result(p, row, m, tok, lp, nk);
    }
    __syncthreads();  // this row's last reads of LDS before the next row's tables
  }
}

// ====================================================================== TOPP
// Top-p without top-k or min-p.  The kept set is the shortest prefix of the (z desc,
// index asc) order whose fixed-point mass reaches top_p_threshold(top_p, total), so the
// total over the whole row is needed before any token can be placed.  The row is read
// two or three times instead of being written to a workspace:
//   1. z of every token (penalties exact), the row maximum and its first index;
//   2. every token's exact mass (mass_of) into the row total; at or above the depth where
//      the boundary can lie (topp_depth), into a bin of the float bits of (zmax - z); and
//      the tokens with d = z - zmax at or above a bound that rises as it fills into an
//      LDS list.  fl(zmax - z) is monotone in z, so the bins split the descending order
//      into consecutive runs.
// The cumulative bin masses then name the bin b* holding the boundary.  Tokens of bins
// before b* are kept (their masses go to the chunk table, one u64 per 64*G-element chunk
// as in FULL, and to the exp sum); the tokens of b* are sorted and kept up to the first
// prefix reaching the threshold.  Both sets come from the list when it covers every bin
// up to b* (the bound stayed below b*'s range), else from a third read.  A b* above
// TOPP_CAP tokens flags the row ST_FALLBACK for generic_kernel.
// The draw scans the chunk table and re-reads one chunk.

// The list's bound on d = z - zmax for a list of c tokens out of cap: it rises as the
// list fills, so rows with many tokens near the maximum keep only the nearest.
__device__ __forceinline__ float topp_list_bound(int c, int cap) {
  const int e = c * 8 / cap;  // eighths of the list in use
  return e < 1 ? (c * 16 < cap ? -16.0f : -12.0f) : e < 2 ? -8.0f : e < 3 ? -6.0f : e < 4 ? -4.0f
       : e < 5 ? -3.0f : e < 6 ? -2.0f : -1.0f;
}

// The depth below which no token can hold the top-p boundary.  A token with
// d = fl(z - zmax) < D weighs floor(2^43 exp32(d)) < 2^43 e^D (1 + 2^-22), so all V of them
// weigh less than 2^43 ((1 - p) - 2^-40) <= (1 - p) S - 8 once
// V e^D (1 + 2^-22) < (1 - p) - 2^-40 (S >= 2^43, the maximum's own mass).  The tokens at
// or above D then weigh more than p S + 8 > ceil(p S): the boundary and every bin before
// it lie at or above D, so the bins need no token below it.  Tokens below -31 weigh 0.
__device__ __forceinline__ float topp_depth(float top_p, int V) {
  const double a = (1.0 - (double)top_p) - 0x1p-40;
  if (!(a > 0.0)) return -31.0f;
  return fmaxf((float)(log(a / ((double)V * 1.0001)) - 0.01), -31.0f);
}

__device__ __forceinline__ int topp_bin(float z, float zmax) {
  const int b = (int)(__float_as_uint(zmax - z) >> 16) - TOPP_BIN_BASE;
  return min(max(b, 0), TOPP_BINS - 1);
}

// NT: TOPP_NT, or 512 where two workgroups fit a CU's LDS (one row's read of the maximum
// then overlaps the other's mass pass)
template <typename TIn, int G, bool VEC, int NT = TOPP_NT>
__global__ __launch_bounds__(NT, 4) void topp_kernel(Params p) {
  constexpr int HR = 4, TILE = NT * G, CH = 64 * G;
  extern __shared__ __align__(16) unsigned char smem[];
  const Layout L = make_layout<MODE_TOPP, G>(p.V, p.words, p.ucap, p.cap);
  Misc* m = reinterpret_cast<Misc*>(smem + L.misc);
  const Hist h = hist_tables(smem, L);
  uint64_t* bins = reinterpret_cast<uint64_t*>(smem + L.mode0);
  uint64_t* chunks = bins + TOPP_BINS;
  const int nch = n_chunks<G>(p.V);
  uint64_t* cand = chunks + nch;

  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  HistIds<HR> hi;
  load_history<NT, HR>(p, row, hi);
  const TIn* src = row_ptr<TIn>(p, row);
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(src, (uint32_t)p.V * (uint32_t)sizeof(TIn));
  const int V = p.V;

  // ---- pass 1: maximum and its first index.  Its loads keep the default cache policy
  // (not the streams' non-temporal one): the second pass reads the same lines tens of
  // microseconds later, and some are still in the Infinity Cache (E's shape, top-p 0.9:
  // 1010 -> 991 us)
  int bad = 0, U = 0;
  float bm = NEG_INF;
  int bi = 0x7FFFFFFF;
  stream_row<TIn, G, NT, VEC, false, 0>(
      p, rs, h,
      [&]() {
        if (tid == 0) {
          m->status = 0;
          m->count = 0;
        }
        for (int i = tid; i < TOPP_BINS; i += NT) bins[i] = 0;
        for (int i = tid; i < nch; i += NT) chunks[i] = 0;
        __syncthreads();
        if (p.has_pen) U = build_history<NT, HR>(p, row, hi, h, m);
        landed(hi);
        return U;
      },
      [&](int t0, int nt, Raw<TIn, G>(&R)[PF], int s0, int n, float gx) {
#pragma unroll
        for (int k = 0; k < PF; ++k) {
          const int t = t0 + k;
          if (t < nt) {
            const int base = t * TILE + tid * G;
            float x[G], z[G];
            unpack(R[k], x);
            make_z<G, true>(x, base, p, h.bitmap, z, bad);
#pragma unroll
            for (int j = 0; j < G; ++j)
              if (z[j] > bm) {
                bm = z[j];
                bi = base + j;
              }
          }
        }
        for (int i = tid; i < n; i += NT) {
          const int s = s0 + i;
          const int tok = (int)h.tok[s];
          const float x = i == tid ? gx : load_one<TIn>(rs, tok);
          const float z = pen_z(x, count_of(h, s), p);
          if (!isfinite(z)) bad = 1;
          if (z > bm || (z == bm && tok < bi)) {
            bm = z;
            bi = tok;
          }
        }
      });
  if (bad) atomicOr(&m->status, ST_NONFINITE);
  const float zmax = block_max<NT>(bm, m);
  int am = block_min_i<NT>(bm == zmax ? bi : 0x7FFFFFFF, m);
  if (am < 0 || am >= V) am = 0;
  const float u = row_uniform(p, row, m);
  __syncthreads();
  if (m->status & ST_NONFINITE) {
    if (tid == 0) write_result(p, row, m, am, 0.0f, 0);
    return;
  }
  const double dmax = (double)zmax;

  // ---- pass 2: exact masses into the row total; tokens at or above the boundary depth
  // dstar into the bins, and those near the maximum into the list.  d = fl(z - zmax) is
  // -fl(zmax - z), the bins' own difference.  A thread lists a token when d >= its bound db,
  // which only rises with the list's length, so the list holds every token with
  // d >= (the largest final db).  A tile's G masses (each at most 2^43) sum exactly in fp64.
  uint64_t tot = 0;
  const float dstar = topp_depth(p.top_p, V);
  float db = fmaxf(-16.0f, dstar);
  int lost = 0;
  auto offer = [&](float z, int idx) {
    const int pos = atomicAdd(&m->count, 1);
    if (pos < p.cap) cand[pos] = ckey(z, (uint32_t)idx);
    else lost = 1;
  };
  auto pass_setup = [&]() { return U; };
  stream_row<TIn, G, NT, VEC, false>(
      p, rs, h, pass_setup,
      [&](int t0, int nt, Raw<TIn, G>(&R)[PF], int s0, int n, float gx) {
#pragma unroll
        for (int k = 0; k < PF; ++k) {
          const int t = t0 + k;
          if (t < nt) {
            const int base = t * TILE + tid * G;
            float x[G], z[G];
            unpack(R[k], x);
            make_z<G, true>(x, base, p, h.bitmap, z, bad);
            double ts = 0.0;
#pragma unroll
            for (int j = 0; j < G; ++j) {
              const float ms = mass_ff(z[j], zmax);
              ts += (double)ms;
              const float d = z[j] - zmax;
              if (d >= dstar && ms != 0.0f) {
                atomicAdd((unsigned long long*)&bins[topp_bin(z[j], zmax)], (unsigned long long)ms);
                if (d >= db) offer(z[j], base + j);
              }
            }
            tot += (uint64_t)ts;
            db = fmaxf(db, topp_list_bound(__atomic_load_n(&m->count, __ATOMIC_RELAXED), p.cap));
          }
        }
        for (int i = tid; i < n; i += NT) {
          const int s = s0 + i;
          const int tok = (int)h.tok[s];
          const float x = i == tid ? gx : load_one<TIn>(rs, tok);
          const float z = pen_z(x, count_of(h, s), p);
          const uint64_t ms = mass_of(z, zmax);
          tot += ms;
          const float d = z - zmax;
          if (d >= dstar && ms != 0) {
            atomicAdd((unsigned long long*)&bins[topp_bin(z, zmax)], (unsigned long long)ms);
            if (d >= db) offer(z, tok);
          }
        }
      });
  tot = block_sum_u64<NT>(tot, m);  // its barriers also order the bin and list atomics
  const uint64_t thr = top_p_threshold(p.top_p, tot);
  const float dbf = block_max<NT>(db, m);
  lost = block_sum_i<NT>(lost, m);
  const int nl = min(m->count, p.cap);

  // bin b* with (mass of bins < b*) < thr <= (mass of bins <= b*); the maximum's own
  // mass (2^43, bin 0) makes it exist for every finite row
  if (wid == 0) {
    if (lane == 0) m->bi[0] = -1;
    constexpr int PER = TOPP_BINS / 64;
    uint64_t s = 0;
    for (int q = 0; q < PER; ++q) s += bins[lane * PER + q];
    const uint64_t incl = wave_incl_scan_u64(s, lane);
    const uint64_t before = incl - s;
    if (before < thr && thr <= incl) {
      uint64_t acc = before;
      for (int q = 0; q < PER; ++q) {
        const uint64_t v = bins[lane * PER + q];
        if (acc + v >= thr) {
          m->bi[0] = lane * PER + q;
          m->bu[0] = acc;
          break;
        }
        acc += v;
      }
    }
  }
  __syncthreads();
  const int bstar = m->bi[0];
  const uint64_t cum_before = m->bu[0];
  if (tid == 0) m->count = 0;
  __syncthreads();

  // The list covers bins <= b* when every token there has d >= dbf: such a token has
  // fl(zmax - z) below the bin's upper edge ub, so d = -fl(zmax - z) > -ub (the test
  // keeps a margin of 2^-22).
  bool from_list = !lost && bstar >= 0 && bstar < TOPP_BINS - 1;
  if (from_list) {
    const float ub = __uint_as_float((uint32_t)(bstar + TOPP_BIN_BASE + 1) << 16);
    from_list = (double)ub * (1.0 + 0x1p-22) <= -(double)dbf;
  }
  // the boundary bin's tokens, unsorted: from the list into the bins' space (free now),
  // or from a third read into the list's space
  uint64_t* blist = from_list ? bins : cand;
  double es = 0.0;
  int nk = 0;
  if (from_list) {
    for (int i = tid; i < nl; i += NT) {
      const uint64_t key = cand[i];
      const float z = ckey_z(key);
      const int b = topp_bin(z, zmax);
      if (b < bstar) {
        const double e = exp_det((double)z - dmax);
        atomicAdd((unsigned long long*)&chunks[ckey_idx(key) / CH], (unsigned long long)mass_of(z, zmax));
        es += e;
        ++nk;
      } else if (b == bstar) {
        blist[atomicAdd(&m->count, 1)] = key;  // at most nl <= TOPP_CAP <= TOPP_BINS
      }
    }
  } else {
    // pass 3: kept masses per chunk, the boundary bin's tokens
    stream_row<TIn, G, NT, VEC, false>(
        p, rs, h, pass_setup,
        [&](int t0, int nt, Raw<TIn, G>(&R)[PF], int s0, int n, float gx) {
#pragma unroll
          for (int k = 0; k < PF; ++k) {
            const int t = t0 + k;
            if (t < nt) {
              const int base = t * TILE + tid * G;
              float x[G], z[G];
              unpack(R[k], x);
              make_z<G, true>(x, base, p, h.bitmap, z, bad);
              uint64_t cs = 0;
#pragma unroll
              for (int j = 0; j < G; ++j) {
                const double d = (double)z[j] - dmax;
                if (d >= -30.0) {
                  const int b = topp_bin(z[j], zmax);
                  if (b < bstar) {
                    const double e = exp_det(d);
                    cs += mass_of(z[j], zmax);
                    es += e;
                    ++nk;
                  } else if (b == bstar) {
                    const int pos = atomicAdd(&m->count, 1);
                    if (pos < p.cap) cand[pos] = ckey(z[j], (uint32_t)(base + j));
                  }
                }
              }
              if (__builtin_amdgcn_ballot_w64(cs != 0)) {
                cs = wave_sum_u64(cs);
                if (lane == 0) atomicAdd((unsigned long long*)&chunks[t * (NT / 64) + wid], (unsigned long long)cs);
              }
            }
          }
          for (int i = tid; i < n; i += NT) {
            const int s = s0 + i;
            const int tok = (int)h.tok[s];
            const float x = i == tid ? gx : load_one<TIn>(rs, tok);
            const float z = pen_z(x, count_of(h, s), p);
            const double d = (double)z - dmax;
            if (d >= -30.0) {
              const int b = topp_bin(z, zmax);
              if (b < bstar) {
                const double e = exp_det(d);
                atomicAdd((unsigned long long*)&chunks[tok / CH], (unsigned long long)mass_of(z, zmax));
                es += e;
                ++nk;
              } else if (b == bstar) {
                const int pos = atomicAdd(&m->count, 1);
                if (pos < p.cap) cand[pos] = ckey(z, (uint32_t)tok);
              }
            }
          }
        });
  }
  __syncthreads();
  const int nc = m->count;
  if (nc > p.cap || bstar < 0) {
    if (tid == 0) p.out_status[row] = m->status | ST_FALLBACK;
    return;
  }
  // the boundary inside b*: the first prefix of its sorted tokens reaching thr
  bitonic_sort_desc<NT>(blist, nc);
  __syncthreads();
  if (wid == 0) {
    uint64_t carry = cum_before;
    int js = nc - 1;
    for (int c0 = 0; c0 < nc; c0 += 64) {
      const int j = c0 + lane;
      const uint64_t ms = j < nc ? mass_of(ckey_z(blist[j]), zmax) : 0;
      const uint64_t incl = wave_incl_scan_u64(ms, lane) + carry;
      const uint64_t hit = __builtin_amdgcn_ballot_w64(j < nc && incl >= thr);
      if (hit) {
        js = c0 + __builtin_ctzll(hit);
        break;
      }
      carry = __shfl(incl, 63);
    }
    if (lane == 0) m->bi[1] = js;
  }
  __syncthreads();
  const int jstar = m->bi[1];

  // kept tokens of b*: blist[0..jstar]; every kept token has key >= blist[jstar]
  for (int j = tid; j <= jstar; j += NT) {
    const uint64_t key = blist[j];
    const double e = exp_det((double)ckey_z(key) - dmax);
    atomicAdd((unsigned long long*)&chunks[ckey_idx(key) / CH], (unsigned long long)mass_of(ckey_z(key), zmax));
    es += e;
    ++nk;
  }
  const uint64_t Bkey = jstar >= 0 && jstar < nc ? blist[jstar] : ~0ull;
  nk = block_sum_i<NT>(nk, m);
  const double esum = block_sum_d<NT>(es, m);  // its barriers also order the chunk atomics

  int64_t tok = am;
  float ztok = zmax;
  if (!p.greedy) {
    uint64_t sk = 0;
    for (int i = tid; i < nch; i += NT) sk += chunks[i];
    sk = block_sum_u64<NT>(sk, m);
    const uint64_t t = draw_target(u, sk);
    block_incl_scan_u64<NT>(chunks, nch, m);
    // first chunk whose inclusive mass exceeds t
    for (int c = tid; c < nch; c += NT) {
      const uint64_t before = c ? chunks[c - 1] : 0;
      if (before <= t && t < chunks[c]) {
        m->bi[2] = c;
        m->bu[1] = before;
      }
    }
    __syncthreads();
    const int c = m->bi[2];
    const uint64_t before = m->bu[1];
    if (wid == 0) {
      // re-read chunk c; kept = bin < b*, or bin b* at or above the boundary key
      const int base = c * CH + lane * G;
      uint64_t ms[G];
      float zz[G];
      uint64_t ls = 0;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const int idx = base + j;
        float z = NEG_INF;
        if (idx < V) {
          const float x = load_one<TIn>(rs, idx);
          if (p.has_pen && ((h.bitmap[idx >> 5] >> (idx & 31)) & 1u)) {
            const int sl = slot_of(h, idx);
            z = pen_z(x, count_of(h, sl), p);
          } else {
            z = div_T(x, p);
          }
        }
        zz[j] = z;
        ms[j] = 0;
        const double d = (double)z - dmax;
        if (d >= -30.0 && ckey(z, (uint32_t)idx) >= Bkey) ms[j] = mass_of(z, zmax);
        ls += ms[j];
      }
      const uint64_t incl = wave_incl_scan_u64(ls, lane) + before;
      uint64_t acc = incl - ls;
      int pick = -1;
      float zp = 0.0f;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        if (pick < 0 && ms[j] != 0 && t < acc + ms[j]) {
          pick = base + j;
          zp = zz[j];
        }
        acc += ms[j];
      }
      const uint64_t hit = __builtin_amdgcn_ballot_w64(pick >= 0);
      if (hit) {
        const int src_lane = __builtin_ctzll(hit);
        const int pk = __shfl(pick, src_lane);
        const float zpk = __shfl(zp, src_lane);
        if (lane == 0) {
          m->bi[3] = pk;
          m->bf[0] = zpk;
        }
      } else if (lane == 0) {
        m->bi[3] = -1;
      }
    }
    __syncthreads();
    if (m->bi[3] >= 0) {
      tok = m->bi[3];
      ztok = m->bf[0];
    }
  }
  if (tid == 0) {
    const float lp = (float)(((double)ztok - dmax) - log(esum));
    write_result(p, row, m, tok, lp, nk);
  }
}

// One wave per deferred TOPK row: the final selection over the row's candidates,
// exactly as topk_kernel runs it in place.  The row's status so far is in out_status.
//
// Every decision of the selection (top-k, top-p, the draw, the log-prob) is taken over
// the candidates that pass min-p against the largest candidate, and those are a prefix
// of the sorted order.  So the wave first keeps only those, in LDS, and sorts 64*R of
// them with R chosen by their count: a row with 150 candidates of which 50 pass min-p
// takes the one-key-per-lane sort.
__global__ __launch_bounds__(SEL_WAVES * 64) void select_kernel(Params p, int rows) {
  __shared__ Misc ms[SEL_WAVES];
  __shared__ uint64_t kept_keys[SEL_WAVES][DEFER_KEYS];
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const int row = blockIdx.x * SEL_WAVES + wid;
  if (row >= rows) return;
  // The row's count, status, uniform and first 64 key slots load together (one round trip
  // instead of three; all DEFER_KEYS slots of a row are allocated, and those past its
  // count are not used).  Most rows hold fewer than 64 keys.
  const uint64_t* keys = p.defer_keys + (int64_t)row * DEFER_KEYS;
  const uint64_t first = keys[lane];
  const int n = p.defer_count[row];
  const int st0 = p.out_status[row];
  const float u0 = p.greedy ? 0.0f : p.uniforms[row];
  if (n < 1 || n > DEFER_KEYS) return;
  Misc* m = &ms[wid];
  if (lane == 0) m->status = st0;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float u = u0;  // as row_uniform
  if (!p.greedy && !(u0 >= 0.0f && u0 < 1.0f)) {
    atomicOr(&m->status, ST_BAD_UNIFORM);
    u = 0.0f;
  }
  constexpr int RK = DEFER_KEYS / 64;
  uint64_t k[RK];
  float zl = NEG_INF;
#pragma unroll
  for (int r = 0; r < RK; ++r) {
    k[r] = r * 64 + lane < n ? (r == 0 ? first : keys[r * 64 + lane]) : 0;  // 0 is below every key
    if (r * 64 + lane < n) zl = fmaxf(zl, ckey_z(k[r]));
  }
  // the row maximum the selection measures min-p against: the largest key's z, which is the
  // largest of the keys' z (the key order puts z first)
  const float zmax = wave_max_dpp(zl);
  uint64_t* buf = kept_keys[wid];
  int el = 0;
#pragma unroll
  for (int r = 0; r < RK; ++r) {
    const bool ok = r * 64 + lane < n && minp_ok(ckey_z(k[r]), zmax, p);
    const unsigned long long b = __ballot(ok);
    if (ok) buf[el + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u))] = k[r];
    el += (int)__popcll(b);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (el <= 64) wave_final<1, true>(p, row, m, buf, el, u);
  else if (el <= 128) wave_final<2, true>(p, row, m, buf, el, u);
  else wave_final<4, true>(p, row, m, buf, el, u);
}

// One workgroup per row of a vocabulary-sharded batch: the final selection over the
// union of the candidate lists the shards emitted (topk_kernel<..., EMIT>), exactly as an
// unsharded row would finish.  The row's status is the OR of the shards' statuses.
// merge_kernel's LDS: Misc, 256 keys of scratch (the lists' counts and offsets, then the
// radix bins) and the candidates: the lists' keys plus top_k, and at least the
// MERGE_TREE_KEYS of the small-top_k merge tree.
constexpr int MERGE_TREE_KEYS = TOPK_NT;
inline size_t merge_lds_bytes(size_t list_keys, int top_k) {
  return align16(sizeof(Misc)) + (256 + std::max(list_keys + (size_t)top_k, (size_t)MERGE_TREE_KEYS)) * sizeof(uint64_t);
}

struct MergeIn {
  const uint64_t* keys;   // [shards, rows, stride]
  const int32_t* counts;  // [shards, rows]
  const int32_t* status;  // [shards, rows]
  int shards, rows, stride;
  int take;  // keys used per list: min(stride, top_k), the size of the LDS buffer's shares
};

__global__ __launch_bounds__(TOPK_NT) void merge_kernel(Params p, MergeIn in) {
  constexpr int NT = TOPK_NT;
  extern __shared__ __align__(16) unsigned char smem[];
  Misc* m = reinterpret_cast<Misc*>(smem);
  uint64_t* hist = reinterpret_cast<uint64_t*>(smem + align16(sizeof(Misc)));
  uint64_t* cand = hist + 256;
  const int row = blockIdx.x, tid = threadIdx.x, wid = tid >> 6;
  if (in.shards <= 256) {
    // every list's count and status at once, their offsets in LDS (hist is free until the
    // compaction), then one flat copy with all loads in flight
    int* cnt = reinterpret_cast<int*>(hist);
    int* off = cnt + 256;
    if (tid == 0) m->status = 0;
    __syncthreads();
    if (tid < in.shards) {
      cnt[tid] = min(max(in.counts[(int64_t)tid * in.rows + row], 0), in.take);
      const int st = in.status[(int64_t)tid * in.rows + row];
      if (st) atomicOr(&m->status, st);
    }
    __syncthreads();
    if (tid == 0) {
      int a = 0;
      for (int s = 0; s < in.shards; ++s) {
        off[s] = a;
        a += cnt[s];
      }
      m->count = a;
    }
    __syncthreads();
    const int tot = in.shards * in.take;
    for (int j = tid; j < tot; j += NT) {
      const int s = j / in.take, i = j - s * in.take;
      if (i < cnt[s]) cand[off[s] + i] = in.keys[((int64_t)s * in.rows + row) * in.stride + i];
    }
  } else {
    if (tid == 0) {
      int st = 0, n = 0;
      for (int s = 0; s < in.shards; ++s) {
        st |= in.status[(int64_t)s * in.rows + row];
        n += min(max(in.counts[(int64_t)s * in.rows + row], 0), in.take);
      }
      m->status = st;
      m->count = n;
    }
    __syncthreads();
    int base = 0;
    for (int s = 0; s < in.shards; ++s) {
      const int c = min(max(in.counts[(int64_t)s * in.rows + row], 0), in.take);
      const uint64_t* src = in.keys + ((int64_t)s * in.rows + row) * in.stride;
      for (int i = tid; i < c; i += NT) cand[base + i] = src[i];
      base += c;
    }
  }
  __syncthreads();
  int n = m->count;
  // top_k <= 64: every list is its slice's top keys sorted descending (the emitting kernel
  // sorts them), so the union's 64 largest keys come from pairwise bitonic merges in
  // registers: each wave merges its lists, then the waves' results merge pairwise through
  // LDS.  The final selection takes the top_k within min-p of the largest key, all of them
  // among these 64, so it decides exactly as over the whole union (measured on config A:
  // 1.5 us here against 8.9 us for the radix selection over its 1100 keys).
  // (Lists from callers of dsv41_sampler_merge_run that are not sorted take the general
  // path below; cand holds at least MERGE_TREE_KEYS keys for the waves' results.)
  if (in.shards <= 256 && p.top_k <= 64 && in.take <= 64 && n > 64) {
    constexpr int NW = NT / 64;
    static_assert(NW * 64 <= MERGE_TREE_KEYS, "merge tree space");
    const int lane = tid & 63;
    const int* cnt = reinterpret_cast<const int*>(hist);
    const int* off = cnt + 256;
    if (tid == 0) m->unsorted = 0;
    __syncthreads();
    uint64_t best = 0;  // 0 is below every key
    int unsorted = 0;
    for (int s = wid; s < in.shards; s += NW) {
      const int c = cnt[s];
      const uint64_t b = 63 - lane < c ? cand[off[s] + 63 - lane] : 0;  // ascending over the lanes if sorted
      unsorted |= b > __shfl_down(b, 1) ? 1 : 0;                           // (lane 63 compares with itself)
      best = wave_merge_top64(best, b, lane);
    }
    if (__ballot(unsorted) && lane == 0) atomicOr(&m->unsorted, 1);
    __syncthreads();  // every list read: cand takes the waves' results
    if (m->unsorted == 0) {
      cand[wid * 64 + lane] = best;
      for (int half = NW / 2; half >= 1; half >>= 1) {
        __syncthreads();
        if (wid < half) {
          best = wave_merge_top64(best, cand[(wid + half) * 64 + 63 - lane], lane);
          cand[wid * 64 + lane] = best;
        }
      }
      if (wid == 0) {
        n = (int)__popcll(__ballot(best != 0));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const float u = row_uniform(p, row, m);
        wave_final<1, true>(p, row, m, cand, n, u);
      }
      return;
    }
  }
  // More keys than one wave sorts: keep the union's top_k within the min-p bound of its
  // largest key, as topk_kernel's own compaction does (every list holds its slice's
  // largest key, so that bound is the row's).  The final selection is the same on the
  // survivors, and the one-wave path then takes any top_k up to 256.
  if (n > 4 * 64) {
    float zl = NEG_INF;
    for (int i = tid; i < n; i += NT) zl = fmaxf(zl, ckey_z(cand[i]));
    const float mz = block_max<NT>(zl, m);
    float tau = NEG_INF;
    uint64_t tau_key = 0;
    n = topk_compact<NT>(cand, n, m, p, mz, tau, tau_key, hist);
  }
  if (n >= 1 && n <= 4 * 64) {
    if (wid == 0) {
      const float u = row_uniform(p, row, m);
      if (n <= 64) wave_final<1, true>(p, row, m, cand, n, u);
      else if (n <= 128) wave_final<2, true>(p, row, m, cand, n, u);
      else wave_final<4, true>(p, row, m, cand, n, u);
    }
    return;
  }
  block_final<NT>(p, row, m, cand, n, hist);
}

// One thread per row of a full-vocabulary draw over slices: the row's maximum and total
// from the gathered states, the token from the picks (inverse CDF: the one slice that
// placed it; race: the best p / E, first id on ties; greedy: the first slice holding the
// maximum), and the outputs as full_kernel writes them.
__global__ __launch_bounds__(256) void full_finish_kernel(dsv41_sampler_full_finish_desc d) {
  const int row = blockIdx.x * 256 + (int)threadIdx.x;
  if (row >= d.rows) return;
  float M;
  double S;
  combine_states(d.states, d.n_shards, d.rows, row, M, S);
  int st = 0;
  for (int s = 0; s < d.n_shards; ++s) st |= d.states[(int64_t)s * d.rows + row].status;
  int64_t tok = 0;
  float ztok = M;
  if (d.draw == DSV41_FULL_DRAW_GREEDY) {
    for (int s = 0; s < d.n_shards; ++s) {
      const dsv41_full_state& x = d.states[(int64_t)s * d.rows + row];
      if (M > NEG_INF && x.max_z == M) {
        tok = x.argmax;
        break;
      }
    }
  } else if (d.draw == DSV41_FULL_DRAW_RACE) {
    float best = -1.0f;
    int64_t bid = INT64_MAX;
    for (int s = 0; s < d.n_shards; ++s) {
      const dsv41_full_pick& pk = d.picks[(int64_t)s * d.rows + row];
      if (pk.id >= 0 && (pk.ratio > best || (pk.ratio == best && pk.id < bid))) {
        best = pk.ratio;
        bid = pk.id;
        ztok = pk.z;
      }
    }
    if (bid != INT64_MAX) tok = bid;
  } else {
    const float u = d.uniforms[row];
    if (!(u >= 0.0f && u < 1.0f)) st |= ST_BAD_UNIFORM;
    bool placed = false;
    for (int s = 0; s < d.n_shards; ++s) {
      const dsv41_full_pick& pk = d.picks[(int64_t)s * d.rows + row];
      if (pk.id >= 0) {
        tok = pk.id;
        ztok = pk.z;
        placed = true;
        break;
      }
    }
    // a finite row always has mass (its maximum weighs 2^43), so some slice places it
    if (!placed && !(st & ST_NONFINITE)) st |= ST_BAD_SLICES;
  }
  if (st & (ST_NONFINITE | ST_BAD_SLICES)) {
    d.out_ids[row] = -1;
    if (d.out_logprob) d.out_logprob[row] = __builtin_nanf("");
    if (d.out_kept) d.out_kept[row] = 0;
  } else {
    d.out_ids[row] = tok;
    if (d.out_logprob) d.out_logprob[row] = (float)(((double)ztok - (double)M) - log(S));
    if (d.out_kept) d.out_kept[row] = (int32_t)d.vocab_size;
  }
  d.out_status[row] = st;
}

// ====================================================================== host
// 256-thread row launches of top_k <= 256 without min-p take topk_kernel<..., SEED>
inline bool topk_seeded(const Params& q, int nt) {
  return nt == 256 && q.top_k >= 1 && q.top_k <= 256 && !(q.min_p > 0.0f);
}

template <class K>
int launch(K kernel, int nt, size_t lds, int rows, const Params& prm, hipStream_t stream) {
  DSV41_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_LIMIT));
  hipLaunchKernelGGL(kernel, dim3(rows), dim3(nt), lds, stream, prm);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}

struct Plan {
  int mode;
  int esize;
  bool vec;
  bool has_pen;
  bool defer;
  bool internal_k;  // TOPK run for min-p without top-k, generic_kernel as the fallback
                    // (TOPP rows fall back to generic_kernel the same way)
  int words, ucap, cap;
  size_t lds;
  size_t workspace;
  int topk_nt;        // TOPK threads per workgroup: TOPK_NT, or 256 (see plan)
  int topp_nt;        // TOPP threads per workgroup: TOPP_NT, or 512 (see plan)
  bool bitmap_only;   // TOPK penalties need only the membership bitmap
  // sliced small TOPK batch (slices > 1): slice width, its table sizes and LDS, the merge's
  // LDS, and the workspace offsets of the slices' keys, counts and statuses
  int slices, slice_w, slice_words, slice_ucap;
  size_t slice_lds, merge_lds, ws_counts, ws_status;
  // small FULL batch over pre_slices slices of pre_sw wave spans per row (full_slice_kernel,
  // pre_lds bytes of history bitmap, + full_kernel<..., PRE>), with the workspace offsets
  // of its arrays
  int pre_slices, pre_sw;
  size_t pre_lds, pre_em, pre_w, pre_st;
};

// shard: the descriptor describes one vocabulary slice (dsv41_sampler_shard_run); the draw
// and the per-row outputs happen in the merge, so uniforms and outputs are not checked here.
int plan(const dsv41_sampler_desc* d, Plan* pl, bool shard = false) {
  if (!d) return fail(DSV41_E_INVALID, "sampler descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_sampler_desc))
    return fail(DSV41_E_ABI, "dsv41_sampler_desc size mismatch (rebuild the binding)");
  if (d->rows <= 0 || d->vocab <= 0)
    return fail(DSV41_E_INVALID, "logits must have shape [rows, vocabulary_size] with both nonzero");
  if (d->vocab > MAX_VOCAB) return fail(DSV41_E_UNSUPPORTED, "vocabulary_size of 2^21 or more is not supported");
  if (d->logits_dtype != DSV41_DTYPE_F32 && d->logits_dtype != DSV41_DTYPE_BF16)
    return fail(DSV41_E_INVALID, "logits dtype must be float32 or bfloat16");
  if (!d->logits || d->logits_row_stride < d->vocab)
    return fail(DSV41_E_INVALID, "logits pointer or row stride is invalid");
  if (!(isfinite(d->temperature) && d->temperature > 0.0f))
    return fail(DSV41_E_INVALID, "temperature must be finite and positive");
  if (!(isfinite(d->repetition_penalty) && d->repetition_penalty > 0.0f))
    return fail(DSV41_E_INVALID, "repetition_penalty must be finite and positive");
  if (!isfinite(d->presence_penalty) || !isfinite(d->frequency_penalty))
    return fail(DSV41_E_INVALID, "presence_penalty and frequency_penalty must be finite");
  if (d->top_k < 0) return fail(DSV41_E_INVALID, "top_k must be nonnegative");
  if (!(d->top_p > 0.0f && d->top_p <= 1.0f)) return fail(DSV41_E_INVALID, "top_p must be in (0, 1]");
  if (!(d->min_p >= 0.0f && d->min_p <= 1.0f)) return fail(DSV41_E_INVALID, "min_p must be in [0, 1]");
  if (!shard && !d->greedy && !d->uniforms && !d->replay_ids)
    return fail(DSV41_E_INVALID, "sampling requires one uniform per row");
  if (!shard && (!d->out_ids || !d->out_status)) return fail(DSV41_E_INVALID, "out_ids and out_status are required");
  if (!shard && d->replay_ids && !d->out_logprob) return fail(DSV41_E_INVALID, "replay_ids need out_logprob");
  const bool pen_on = d->repetition_penalty != 1.0f || d->presence_penalty != 0.0f || d->frequency_penalty != 0.0f;
  const bool hist_given = d->history != nullptr && (d->history_lens != nullptr || d->hist_len > 0);
  if (hist_given) {
    if (d->history_row_stride <= 0 || d->history_row_stride > (1 << 27))
      return fail(DSV41_E_INVALID, "history row stride must be in [1, 2^27]");
    if (!d->history_lens && (d->hist_len < 0 || d->hist_len > d->history_row_stride))
      return fail(DSV41_E_INVALID, "hist_len must be within the history row stride");
  }
  pl->has_pen = pen_on && hist_given;
  pl->esize = d->logits_dtype == DSV41_DTYPE_F32 ? 4 : 2;
  // Vector loads also need each row's valid bytes to end on a 16-byte boundary: the buffer
  // range check zeroes a dword that reaches past the row, so a row ending inside a vector
  // (a view of a padded vocabulary, a vocabulary slice) would read its last ids as zero.
  pl->vec = ((uintptr_t)d->logits % 16 == 0) && ((d->logits_row_stride * pl->esize) % 16 == 0) &&
            (((int64_t)d->vocab * pl->esize) % 16 == 0);
  const int V = d->vocab;
  const bool truncating = d->min_p > 0.0f || (d->top_k > 0 && d->top_k < V) || d->top_p < 1.0f;
  if (d->exponentials && truncating)
    return fail(DSV41_E_UNSUPPORTED, "exponential race draws need the full-vocabulary distribution (no top-k, top-p or min-p)");
  if (d->exponentials && d->exponentials_row_stride < d->vocab)
    return fail(DSV41_E_INVALID, "exponentials row stride must be >= vocab");
  if (d->replay_ids && (truncating || d->exponentials || shard))
    return fail(DSV41_E_UNSUPPORTED, "replay_ids take the full-vocabulary distribution (no top-k, top-p, min-p or exponentials)");
  // a vocabulary slice takes the TOPK kernel for any 1 <= top_k <= 2048: at or above the
  // slice width its buffer (top_k + 2048 keys) never compacts and it emits every survivor
  // of the local min-p bound
  if (shard && d->top_k >= 1 && d->top_k <= KCAP) pl->mode = MODE_TOPK;
  else if (!truncating) pl->mode = MODE_FULL;
  else if (d->top_k > 0 && d->top_k < V && d->top_k <= KCAP) pl->mode = MODE_TOPK;
  else pl->mode = MODE_GENERIC;
  // min-p keeps the tokens near the row maximum: usually far fewer than INTERNAL_K, which
  // TOPK handles exactly; rows that would need more go to generic_kernel
  pl->internal_k = !shard && pl->mode == MODE_GENERIC && d->min_p > 0.0f && (d->top_k == 0 || d->top_k >= V) &&
                   V > INTERNAL_K;
  if (pl->internal_k) pl->mode = MODE_TOPK;
  const int k_eff = pl->internal_k ? INTERNAL_K : d->top_k;
  pl->words = pl->has_pen ? (V + 31) / 32 : 0;
  pl->ucap = pl->has_pen ? (int)std::min<int64_t>(d->history_row_stride, V) : 0;
  if (pl->ucap > MAX_UNIQUE)
    return fail(DSV41_E_UNSUPPORTED, "history longer than 65535 ids per row is not supported");
  // top-p alone: three streams of the row (topp_kernel) where its tables fit on chip
  if (!shard && pl->mode == MODE_GENERIC && d->top_p < 1.0f && !(d->min_p > 0.0f) &&
      (d->top_k == 0 || d->top_k >= V) &&
      make_layout<MODE_TOPP, 4>(V, pl->words, pl->ucap, TOPP_CAP).total <= LDS_LIMIT)
    pl->mode = MODE_TOPP;
  pl->cap = pl->mode == MODE_TOPK ? k_eff + TOPK_TILE : pl->mode == MODE_TOPP ? TOPP_CAP : 0;
  Layout L;
  if (pl->mode == MODE_FULL)
    L = make_layout<MODE_FULL, 8>(V, pl->words, pl->ucap, 0);  // the same for 4 or 8 logits per lane
  else if (pl->mode == MODE_TOPK)
    L = make_layout<MODE_TOPK, TOPK_G>(V, pl->words, pl->ucap, pl->cap);
  else if (pl->mode == MODE_TOPP)
    L = make_layout<MODE_TOPP, 4>(V, pl->words, pl->ucap, pl->cap);
  else
    L = make_layout<MODE_GENERIC, 4>(V, pl->words, pl->ucap, 0);
  pl->lds = L.total;
  if (pl->lds > LDS_LIMIT)
    return fail(DSV41_E_UNSUPPORTED, "history length and vocabulary exceed the on-chip penalty tables");
  pl->defer = !shard && pl->mode == MODE_TOPK && d->rows > DEFER_MIN_ROWS;
  // Batches of at least two rows per CU whose TOPP tables fit two workgroups per CU run
  // with 512 threads: a row's first read (memory) then overlaps another's mass pass (ALU).
  pl->topp_nt = pl->mode == MODE_TOPP && d->rows >= 512 && 2 * pl->lds <= LDS_LIMIT ? 512 : TOPP_NT;
  // Deferred TOPK batches whose tables fit four 256-thread workgroups per CU (a quarter of
  // LDS) run with 256 threads: 128 VGPRs then hold four rows per CU instead of two, so a
  // row building its history tables leaves three others streaming.  Lowering penalties
  // without a frequency penalty need only the membership bitmap.
  pl->topk_nt = TOPK_NT;
  pl->bitmap_only = pl->has_pen && d->repetition_penalty >= 1.0f && d->presence_penalty >= 0.0f &&
                    d->frequency_penalty == 0.0f && !(d->history_prompt_lens && d->presence_penalty != 0.0f);
  if (pl->defer) {
    const int cap256 = k_eff + 256 * TOPK_G;
    const Layout L256 = make_layout<MODE_TOPK, TOPK_G>(V, pl->words, pl->bitmap_only ? 0 : pl->ucap, cap256,
                                                       !pl->bitmap_only);
    if (4 * L256.total <= LDS_LIMIT) {
      pl->topk_nt = 256;
      pl->cap = cap256;
      pl->lds = L256.total;
    }
  }
  pl->workspace = 0;
  if (pl->defer) pl->workspace += (size_t)d->rows * (DEFER_KEYS * sizeof(uint64_t) + sizeof(int32_t));
  // A top-k batch too small to fill the GPU (no deferral, no internal bound) is spread over
  // it: about 256 workgroups, each one tile-aligned slice of a row emitting its exact local
  // top_k, then the merge.  The union of the slices' lists holds each row's kept set.
  pl->slices = 1;
  if (!shard && pl->mode == MODE_TOPK && !pl->defer && !pl->internal_k && d->top_k <= 256) {
    // the merge holds at most 4096 candidates per row.  A slice spans at least three
    // tiles: a slice's first tile fills the buffer before any threshold exists, so two
    // compactions of about 2048 keys come with every slice, and on one or two tiles they
    // outweigh the stream (measured: 4096-id slices slower than 6144-id ones)
    const int want = std::min(std::max(1, 256 / d->rows), 4096 / std::max(1, d->top_k));
    const int sw = std::max(3 * TOPK_TILE,
                            (int)((((int64_t)V + want - 1) / want + TOPK_TILE - 1) / TOPK_TILE * TOPK_TILE));
    const int S = (V + sw - 1) / sw;
    if (S >= 2) {
      const int sw_words = pl->has_pen ? (sw + 31) / 32 : 0;
      const int sw_ucap = pl->has_pen ? (int)std::min<int64_t>(d->history_row_stride, sw) : 0;
      const Layout Ls = make_layout<MODE_TOPK, TOPK_G>(sw, sw_words, sw_ucap, d->top_k + TOPK_TILE);
      const size_t mlds = merge_lds_bytes((size_t)S * d->top_k, d->top_k);
      if (Ls.total <= LDS_LIMIT && mlds <= LDS_LIMIT) {
        pl->slices = S;
        pl->slice_w = sw;
        pl->slice_words = sw_words;
        pl->slice_ucap = sw_ucap;
        pl->slice_lds = Ls.total;
        pl->merge_lds = mlds;
        const size_t n = (size_t)S * d->rows;
        pl->ws_counts = n * d->top_k * sizeof(uint64_t);
        pl->ws_status = pl->ws_counts + n * sizeof(int32_t);
        pl->workspace = pl->ws_status + n * sizeof(int32_t);
      }
    }
  }
  // A FULL batch of at most PRE_MAX_ROWS rows leaves most CUs idle with one workgroup per
  // row: about 512 workgroups then each take a run of a row's wave spans (full_slice_kernel,
  // with its range's history bitmap in LDS), and one workgroup per row finishes it from
  // their statistics.
  pl->pre_slices = 0;
  pl->pre_lds = 0;
  if (!shard && pl->mode == MODE_FULL && !d->replay_ids && !d->exponentials && d->rows <= PRE_MAX_ROWS) {
    const int G = pl->esize == 4 ? 4 : 8;  // the spread small batches take 4 fp32 logits per lane
    const int NC = (V + 64 * G - 1) / (64 * G), NE = n_mass_chunks(V);
    const int want = std::max(2, 512 / d->rows);
    const int sw = std::max(PRE_NT / 64, (NC + want - 1) / want);  // at least one span per wave
    const int S = (NC + sw - 1) / sw;
    const size_t slds = pl->has_pen ? (size_t)sw * 2 * G * sizeof(uint32_t) : 0;
    if (S >= 2 && slds <= PRE_MAX_LDS) {
      pl->pre_slices = S;
      pl->pre_sw = sw;
      pl->pre_lds = slds;
      size_t off = align16(pl->workspace);
      pl->pre_em = off;
      off = align16(off + (size_t)d->rows * NE * sizeof(float));
      pl->pre_w = off;
      off = align16(off + (size_t)d->rows * NE * sizeof(uint64_t));
      pl->pre_st = off;
      pl->workspace = off + (size_t)d->rows * S * sizeof(int32_t);
    }
  }
  if (pl->mode == MODE_GENERIC || pl->mode == MODE_TOPP || pl->internal_k) {
    pl->workspace = align16(pl->workspace);  // the z rows follow the hand-over area
    pl->workspace += (size_t)d->rows * (size_t)V * sizeof(float);
    Layout Lg = make_layout<MODE_GENERIC, 4>(V, pl->words, pl->ucap, 0);
    if (Lg.total > LDS_LIMIT)
      return fail(DSV41_E_UNSUPPORTED, "history length and vocabulary exceed the on-chip penalty tables");
  }
  return DSV41_OK;
}

Params make_params(const dsv41_sampler_desc* d, const Plan& pl, void* workspace) {
  Params p{};
  p.logits = d->logits;
  p.lstride = d->logits_row_stride;
  p.hist = d->history;
  p.hstride = d->history_row_stride;
  p.hlens = d->history_lens;
  p.plens = d->history_prompt_lens;
  p.uniforms = d->uniforms;
  p.out_ids = d->out_ids;
  p.out_lp = d->out_logprob;
  p.out_kept = d->out_kept;
  p.out_status = d->out_status;
  p.zbuf = static_cast<float*>(workspace);
  if (pl.defer && pl.internal_k)  // the z rows of the fallback follow the hand-over area
    p.zbuf = reinterpret_cast<float*>(static_cast<char*>(workspace) +
                                      align16((size_t)d->rows * (DEFER_KEYS * sizeof(uint64_t) + sizeof(int32_t))));
  p.exps = d->exponentials;
  p.estride = d->exponentials_row_stride;
  p.replay = d->replay_ids;
  p.log_min_p = d->min_p > 0.0f ? std::log((double)d->min_p) : -INFINITY;
  {
    // log(min_p) as a float rounded toward -inf, for the conservative in-stream bound
    float lf = (float)p.log_min_p;
    if ((double)lf > p.log_min_p) lf = std::nextafter(lf, -INFINITY);
    p.lmin_f = d->min_p > 0.0f ? lf : -INFINITY;
  }
  p.T = d->temperature;
  p.rT = 1.0f / d->temperature;
  p.rp = d->repetition_penalty;
  p.pres = d->presence_penalty;
  p.freq = d->frequency_penalty;
  p.top_p = d->top_p;
  p.min_p = d->min_p;
  p.V = d->vocab;
  p.hlen = d->hist_len;
  p.top_k = pl.internal_k ? INTERNAL_K : d->top_k;
  p.topk_internal = pl.internal_k ? 1 : 0;
  // Seeded 256-thread batches of a small top_k compact sooner: their threshold rises only
  // at a compaction, and below top_k 128 a fresher threshold saves more passers than the
  // extra compactions cost (E's shape: top-k 50 563 -> 534 us with top_k + 64 instead of
  // 2 top_k + 128; top-k 200 and 256 measured slower with the lower trigger).
  p.mid_trigger = pl.internal_k ? INT_MAX
                  : topk_seeded(p, pl.topk_nt) && d->top_k < 128 ? d->top_k + std::min(std::max(d->top_k, 32), 64)
                                                                 : 2 * d->top_k + 128;
  p.greedy = d->greedy ? 1 : 0;
  p.has_pen = pl.has_pen ? 1 : 0;
  p.pen_lowers = pl.has_pen && d->repetition_penalty >= 1.0f && d->presence_penalty >= 0.0f &&
                 d->frequency_penalty >= 0.0f ? 1 : 0;
  p.pen_counts = pl.has_pen && (d->frequency_penalty != 0.0f ||
                                (d->history_prompt_lens && d->presence_penalty != 0.0f)) ? 1 : 0;
  // z = x / T by the three-operation scheme needs x / T normal and finite for
  // 2^-100 <= |x| < 2^100, which holds for T in [2^-20, 2^20]; other temperatures
  // take IEEE division for every element.
  p.fast_div = (d->temperature >= 0x1p-20f && d->temperature <= 0x1p20f) ? 1 : 0;
  p.unit_T = d->temperature == 1.0f ? 1 : 0;
  p.ucap = pl.ucap;
  p.words = pl.words;
  p.cap = pl.cap;
  if (pl.defer) {
    p.defer = 1;
    p.defer_keys = static_cast<uint64_t*>(workspace);
    p.defer_count = reinterpret_cast<int32_t*>(static_cast<char*>(workspace) +
                                               (size_t)d->rows * DEFER_KEYS * sizeof(uint64_t));
  }
  p.voff = 0;
  p.vfull = d->vocab;
  if (pl.pre_slices) {
    char* ws = static_cast<char*>(workspace);
    p.n_slices = pl.pre_slices;
    p.slice_w = pl.pre_sw;
    p.pre_em = reinterpret_cast<float*>(ws + pl.pre_em);
    p.pre_w = reinterpret_cast<uint64_t*>(ws + pl.pre_w);
    p.pre_st = reinterpret_cast<int32_t*>(ws + pl.pre_st);
  }
  return p;
}

}  // namespace sampler
}  // namespace dsv41

using namespace dsv41;
using namespace dsv41::sampler;

extern "C" size_t dsv41_sampler_workspace_bytes(const dsv41_sampler_desc* d) {
  Plan pl;
  if (plan(d, &pl) != DSV41_OK) return 0;
  return pl.workspace;
}

// A small top-k batch spread over the GPU: each (row, slice) workgroup emits its exact
// local top_k into the workspace, then merge_kernel finishes every row.
static int run_sliced(const dsv41_sampler_desc* d, const Plan& pl, const Params& p, char* ws, hipStream_t s) {
  Params q = p;
  q.words = pl.slice_words;
  q.ucap = pl.slice_ucap;
  q.cap = d->top_k + TOPK_TILE;
  q.voff = 0;
  q.vfull = d->vocab;
  q.n_slices = pl.slices;
  q.slice_w = pl.slice_w;
  q.nrows = d->rows;
  q.emit_cap = d->top_k;
  q.emit_keys = reinterpret_cast<uint64_t*>(ws);
  q.emit_count = reinterpret_cast<int32_t*>(ws + pl.ws_counts);
  q.out_status = reinterpret_cast<int32_t*>(ws + pl.ws_status);
  const int grid = d->rows * pl.slices;
  int rc;
  if (pl.esize == 2) rc = pl.vec ? launch(topk_kernel<uint16_t, true, true, TOPK_NT, true>, TOPK_NT, pl.slice_lds, grid, q, s)
                                 : launch(topk_kernel<uint16_t, false, true, TOPK_NT, true>, TOPK_NT, pl.slice_lds, grid, q, s);
  else rc = pl.vec ? launch(topk_kernel<float, true, true, TOPK_NT, true>, TOPK_NT, pl.slice_lds, grid, q, s)
                   : launch(topk_kernel<float, false, true, TOPK_NT, true>, TOPK_NT, pl.slice_lds, grid, q, s);
  if (rc != DSV41_OK) return rc;
  Params m{};
  m.uniforms = d->uniforms;
  m.out_ids = d->out_ids;
  m.out_lp = d->out_logprob;
  m.out_kept = d->out_kept;
  m.out_status = d->out_status;
  m.log_min_p = p.log_min_p;
  m.min_p = d->min_p;
  m.top_p = d->top_p;
  m.top_k = d->top_k;
  m.greedy = d->greedy ? 1 : 0;
  MergeIn in{q.emit_keys, q.emit_count, q.out_status, pl.slices, d->rows, d->top_k, d->top_k};
  DSV41_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(merge_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_LIMIT));
  hipLaunchKernelGGL(merge_kernel, dim3(d->rows), dim3(TOPK_NT), pl.merge_lds, s, m, in);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}

// Rows flagged ST_FALLBACK by topk_kernel (more min-p survivors than the internal bound)
// or topp_kernel (a boundary bin above TOPP_CAP) again, with generic_kernel: at most
// FALLBACK_GRID workgroups read the statuses and redo the flagged rows.
static int run_flagged(const dsv41_sampler_desc* d, const Plan& pl, const Params& p, hipStream_t s) {
  Params g = p;
  g.top_k = d->top_k;
  g.topk_internal = 0;
  g.only_flagged = 1;
  g.nrows = d->rows;
  g.defer = 0;
  g.cap = 0;
  const size_t lds = make_layout<MODE_GENERIC, 4>(d->vocab, pl.words, pl.ucap, 0).total;
  const int grid = std::min(d->rows, FALLBACK_GRID);
  if (pl.esize == 2) return pl.vec ? launch(generic_kernel<uint16_t, 4, true>, GEN_NT, lds, grid, g, s)
                                   : launch(generic_kernel<uint16_t, 4, false>, GEN_NT, lds, grid, g, s);
  return pl.vec ? launch(generic_kernel<float, 4, true>, GEN_NT, lds, grid, g, s)
                : launch(generic_kernel<float, 4, false>, GEN_NT, lds, grid, g, s);
}

// A small FULL batch: the slices' statistics, then one finishing workgroup per row.
// One workgroup per row of a top-k batch: the instantiation without gathered-slot code when
// the batch gathers no history slots (no penalties, or lowering penalties).
template <typename TIn, bool VEC, int NT>
static int launch_topk_rows(size_t lds, int rows, const Params& q, hipStream_t s) {
  const bool gather = q.has_pen && !q.pen_lowers;
  if constexpr (NT == 256) {
    if (topk_seeded(q, NT))
      return gather ? launch(topk_kernel<TIn, VEC, false, NT, false, true, true>, NT, lds, rows, q, s)
                    : launch(topk_kernel<TIn, VEC, false, NT, false, false, true>, NT, lds, rows, q, s);
  }
  if (gather) return launch(topk_kernel<TIn, VEC, false, NT>, NT, lds, rows, q, s);
  return launch(topk_kernel<TIn, VEC, false, NT, false, false>, NT, lds, rows, q, s);
}

static int run_presliced(const dsv41_sampler_desc* d, const Plan& pl, const Params& p, hipStream_t s) {
  const dim3 grid(d->rows * pl.pre_slices), block(PRE_NT);
  const bool bf = pl.esize == 2, ex = !p.greedy, lp = p.out_lp != nullptr;
  // the history bitmap (at most PRE_MAX_LDS bytes) stays under the default dynamic LDS
  // limit: no attribute to raise
  const size_t sl = pl.pre_lds;
  if (bf) {
    if (lp) {
      if (pl.vec) hipLaunchKernelGGL((full_slice_kernel<uint16_t, 8, true>), grid, block, sl, s, p);
      else hipLaunchKernelGGL((full_slice_kernel<uint16_t, 8, false>), grid, block, sl, s, p);
    } else {
      if (pl.vec) hipLaunchKernelGGL((full_slice_kernel<uint16_t, 8, true, false>), grid, block, sl, s, p);
      else hipLaunchKernelGGL((full_slice_kernel<uint16_t, 8, false, false>), grid, block, sl, s, p);
    }
  } else {
    if (lp) {
      if (pl.vec) hipLaunchKernelGGL((full_slice_kernel<float, 4, true>), grid, block, sl, s, p);
      else hipLaunchKernelGGL((full_slice_kernel<float, 4, false>), grid, block, sl, s, p);
    } else {
      if (pl.vec) hipLaunchKernelGGL((full_slice_kernel<float, 4, true, false>), grid, block, sl, s, p);
      else hipLaunchKernelGGL((full_slice_kernel<float, 4, false, false>), grid, block, sl, s, p);
    }
  }
  DSV41_HIP_CHECK(hipGetLastError());
  if (bf) {
    if (ex) return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW_CDF, true>, FULL_NT, pl.lds, d->rows, p, s)
                          : launch(full_kernel<uint16_t, 8, false, DRAW_CDF, true>, FULL_NT, pl.lds, d->rows, p, s);
    if (!lp) return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW_ARGMAX, true>, FULL_NT, pl.lds, d->rows, p, s)
                           : launch(full_kernel<uint16_t, 8, false, DRAW_ARGMAX, true>, FULL_NT, pl.lds, d->rows, p, s);
    return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW_GREEDY, true>, FULL_NT, pl.lds, d->rows, p, s)
                  : launch(full_kernel<uint16_t, 8, false, DRAW_GREEDY, true>, FULL_NT, pl.lds, d->rows, p, s);
  }
  if (ex) return pl.vec ? launch(full_kernel<float, 4, true, DRAW_CDF, true>, FULL_NT, pl.lds, d->rows, p, s)
                        : launch(full_kernel<float, 4, false, DRAW_CDF, true>, FULL_NT, pl.lds, d->rows, p, s);
  if (!lp) return pl.vec ? launch(full_kernel<float, 4, true, DRAW_ARGMAX, true>, FULL_NT, pl.lds, d->rows, p, s)
                         : launch(full_kernel<float, 4, false, DRAW_ARGMAX, true>, FULL_NT, pl.lds, d->rows, p, s);
  return pl.vec ? launch(full_kernel<float, 4, true, DRAW_GREEDY, true>, FULL_NT, pl.lds, d->rows, p, s)
                : launch(full_kernel<float, 4, false, DRAW_GREEDY, true>, FULL_NT, pl.lds, d->rows, p, s);
}

// The launches of one planned batch; `workspace` holds at least pl.workspace bytes.
static int run_planned(const dsv41_sampler_desc* d, const Plan& pl, void* workspace, void* stream) {
  int rc;
  Params p = make_params(d, pl, workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = pl.esize == 2;
  switch (pl.mode) {
    case MODE_FULL:
      if (pl.pre_slices) return run_presliced(d, pl, p, s);
      if (p.replay) {
        if (bf) return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW_REPLAY>, FULL_NT, pl.lds, d->rows, p, s)
                              : launch(full_kernel<uint16_t, 8, false, DRAW_REPLAY>, FULL_NT, pl.lds, d->rows, p, s);
        return pl.vec ? launch(full_kernel<float, 8, true, DRAW_REPLAY>, FULL_NT, pl.lds, d->rows, p, s)
                      : launch(full_kernel<float, 8, false, DRAW_REPLAY>, FULL_NT, pl.lds, d->rows, p, s);
      }
      if (p.greedy && !p.out_lp) {
        if (bf) return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW_ARGMAX>, FULL_NT, pl.lds, d->rows, p, s)
                              : launch(full_kernel<uint16_t, 8, false, DRAW_ARGMAX>, FULL_NT, pl.lds, d->rows, p, s);
        return pl.vec ? launch(full_kernel<float, 4, true, DRAW_ARGMAX>, FULL_NT, pl.lds, d->rows, p, s)
                      : launch(full_kernel<float, 4, false, DRAW_ARGMAX>, FULL_NT, pl.lds, d->rows, p, s);
      }
      if (p.greedy) {
        if (bf) return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW_GREEDY>, FULL_NT, pl.lds, d->rows, p, s)
                              : launch(full_kernel<uint16_t, 8, false, DRAW_GREEDY>, FULL_NT, pl.lds, d->rows, p, s);
        return pl.vec ? launch(full_kernel<float, 8, true, DRAW_GREEDY>, FULL_NT, pl.lds, d->rows, p, s)
                      : launch(full_kernel<float, 8, false, DRAW_GREEDY>, FULL_NT, pl.lds, d->rows, p, s);
      }
      if (p.exps) {
        if (bf) return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW_RACE>, FULL_NT, pl.lds, d->rows, p, s)
                              : launch(full_kernel<uint16_t, 8, false, DRAW_RACE>, FULL_NT, pl.lds, d->rows, p, s);
        return pl.vec ? launch(full_kernel<float, 8, true, DRAW_RACE>, FULL_NT, pl.lds, d->rows, p, s)
                      : launch(full_kernel<float, 8, false, DRAW_RACE>, FULL_NT, pl.lds, d->rows, p, s);
      }
      if (bf) return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW_CDF>, FULL_NT, pl.lds, d->rows, p, s)
                            : launch(full_kernel<uint16_t, 8, false, DRAW_CDF>, FULL_NT, pl.lds, d->rows, p, s);
      return pl.vec ? launch(full_kernel<float, 8, true, DRAW_CDF>, FULL_NT, pl.lds, d->rows, p, s)
                    : launch(full_kernel<float, 8, false, DRAW_CDF>, FULL_NT, pl.lds, d->rows, p, s);
    case MODE_TOPK: {
      if (pl.slices > 1) return run_sliced(d, pl, p, static_cast<char*>(workspace), s);
      if (pl.topk_nt == 256) {
        Params q = p;
        if (pl.bitmap_only) {
          q.ucap = 0;
          q.no_ranks = 1;
        }
        if (bf) rc = pl.vec ? launch_topk_rows<uint16_t, true, 256>(pl.lds, d->rows, q, s)
                            : launch_topk_rows<uint16_t, false, 256>(pl.lds, d->rows, q, s);
        else rc = pl.vec ? launch_topk_rows<float, true, 256>(pl.lds, d->rows, q, s)
                         : launch_topk_rows<float, false, 256>(pl.lds, d->rows, q, s);
      } else if (bf) {
        rc = pl.vec ? launch_topk_rows<uint16_t, true, TOPK_NT>(pl.lds, d->rows, p, s)
                    : launch_topk_rows<uint16_t, false, TOPK_NT>(pl.lds, d->rows, p, s);
      } else {
        rc = pl.vec ? launch_topk_rows<float, true, TOPK_NT>(pl.lds, d->rows, p, s)
                    : launch_topk_rows<float, false, TOPK_NT>(pl.lds, d->rows, p, s);
      }
      if (rc != DSV41_OK) return rc;
      if (pl.defer) {
        hipLaunchKernelGGL(select_kernel, dim3((d->rows + SEL_WAVES - 1) / SEL_WAVES), dim3(SEL_WAVES * 64), 0, s,
                           p, d->rows);
        DSV41_HIP_CHECK(hipGetLastError());
      }
      if (!pl.internal_k) return DSV41_OK;
      return run_flagged(d, pl, p, s);
    }
    case MODE_TOPP:
      if (pl.topp_nt == 512) {
        if (bf) rc = pl.vec ? launch(topp_kernel<uint16_t, 4, true, 512>, 512, pl.lds, d->rows, p, s)
                            : launch(topp_kernel<uint16_t, 4, false, 512>, 512, pl.lds, d->rows, p, s);
        else rc = pl.vec ? launch(topp_kernel<float, 4, true, 512>, 512, pl.lds, d->rows, p, s)
                         : launch(topp_kernel<float, 4, false, 512>, 512, pl.lds, d->rows, p, s);
      } else if (bf) {
        rc = pl.vec ? launch(topp_kernel<uint16_t, 4, true>, TOPP_NT, pl.lds, d->rows, p, s)
                    : launch(topp_kernel<uint16_t, 4, false>, TOPP_NT, pl.lds, d->rows, p, s);
      } else {
        rc = pl.vec ? launch(topp_kernel<float, 4, true>, TOPP_NT, pl.lds, d->rows, p, s)
                    : launch(topp_kernel<float, 4, false>, TOPP_NT, pl.lds, d->rows, p, s);
      }
      if (rc != DSV41_OK) return rc;
      return run_flagged(d, pl, p, s);
    default:
      if (bf) return pl.vec ? launch(generic_kernel<uint16_t, 4, true>, GEN_NT, pl.lds, d->rows, p, s)
                            : launch(generic_kernel<uint16_t, 4, false>, GEN_NT, pl.lds, d->rows, p, s);
      return pl.vec ? launch(generic_kernel<float, 4, true>, GEN_NT, pl.lds, d->rows, p, s)
                    : launch(generic_kernel<float, 4, false>, GEN_NT, pl.lds, d->rows, p, s);
  }
}

extern "C" int dsv41_sampler_run(const dsv41_sampler_desc* d, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  Plan pl;
  const int rc = plan(d, &pl);
  if (rc != DSV41_OK) return rc;
  if (pl.workspace && (!workspace || workspace_bytes < pl.workspace))
    return fail(DSV41_E_WORKSPACE, "sampler workspace is missing or too small");
  return run_planned(d, pl, workspace, stream);
}

// ------------------------------------------------------------ static scratch
// The workspace of dsv41_sampler_run_static: one array per GPU, part of the code object's
// device memory, held until the process ends.  On the host `scratch` names a stand-in, not
// a device address: host code uses the per-device address hipGetSymbolAddress returns.
static __device__ __align__(256) unsigned char scratch[DSV41_SAMPLER_STATIC_SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES];

// The scratch address on the current device, looked up once per device (with that device
// current).  The stream must belong to the current device.
int scratch_address(hipStream_t s, void** out) {
  int dev = 0;
  DSV41_HIP_CHECK(hipGetDevice(&dev));
  if (s) {
    hipDevice_t sdev = 0;
    DSV41_HIP_CHECK(hipStreamGetDevice(s, &sdev));
    if ((int)sdev != dev) return fail(DSV41_E_INVALID, "the stream must belong to the current device");
  }
  if (dev < 0 || dev >= MAX_DEVICES) return fail(DSV41_E_UNSUPPORTED, "device index above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    DSV41_HIP_CHECK(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
    if (!ptr) return fail(DSV41_E_HIP, "hipGetSymbolAddress returned no address for the sampler scratch");
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return DSV41_OK;
}
}  // namespace

extern "C" int dsv41_sampler_run_static(const dsv41_sampler_desc* d, void* stream) {
  Plan pl;
  int rc = plan(d, &pl);
  if (rc != DSV41_OK) return rc;
  if (pl.workspace > (size_t)DSV41_SAMPLER_STATIC_SCRATCH_BYTES)
    return fail(DSV41_E_UNSUPPORTED, "this batch needs " + std::to_string(pl.workspace) +
                                         " bytes of scratch, above the static maximum of " +
                                         std::to_string((size_t)DSV41_SAMPLER_STATIC_SCRATCH_BYTES) +
                                         " (use dsv41_sampler_run with a workspace)");
  void* ws = nullptr;
  rc = scratch_address(static_cast<hipStream_t>(stream), &ws);
  if (rc != DSV41_OK) return rc;
  return run_planned(d, pl, ws, stream);
}

extern "C" int dsv41_sampler_shard_run(const dsv41_sampler_shard_desc* d, void* stream) {
  if (!d) return fail(DSV41_E_INVALID, "sampler shard descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_sampler_shard_desc))
    return fail(DSV41_E_ABI, "dsv41_sampler_shard_desc size mismatch (rebuild the binding)");
  const dsv41_sampler_desc* sd = d->sampler;
  if (!sd) return fail(DSV41_E_INVALID, "sampler shard: the slice's sampler descriptor is NULL");
  Plan pl;
  int rc = plan(sd, &pl, true);
  if (rc != DSV41_OK) return rc;
  if (sd->exponentials) return fail(DSV41_E_UNSUPPORTED, "sampler shard: exponential race draws are not sharded");
  if (pl.mode != MODE_TOPK)
    return fail(DSV41_E_UNSUPPORTED, "vocabulary-sharded sampling needs 1 <= top_k <= 2048");
  if (d->vocab_offset < 0 || d->vocab_size < d->vocab_offset + sd->vocab || d->vocab_size > MAX_VOCAB)
    return fail(DSV41_E_INVALID, "sampler shard: the slice must lie within a vocabulary of fewer than 2^21 ids");
  if (d->max_candidates < sd->top_k) return fail(DSV41_E_INVALID, "sampler shard: max_candidates must be >= top_k");
  if (!d->out_keys || !d->out_counts || !d->out_status)
    return fail(DSV41_E_INVALID, "sampler shard: out_keys, out_counts and out_status are required");
  Params p = make_params(sd, pl, nullptr);
  p.voff = (int)d->vocab_offset;
  p.vfull = (int)d->vocab_size;
  p.emit_cap = d->max_candidates;
  p.emit_keys = d->out_keys;
  p.emit_count = d->out_counts;
  p.out_status = d->out_status;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pl.esize == 2)
    return pl.vec ? launch(topk_kernel<uint16_t, true, true>, TOPK_NT, pl.lds, sd->rows, p, s)
                  : launch(topk_kernel<uint16_t, false, true>, TOPK_NT, pl.lds, sd->rows, p, s);
  return pl.vec ? launch(topk_kernel<float, true, true>, TOPK_NT, pl.lds, sd->rows, p, s)
                : launch(topk_kernel<float, false, true>, TOPK_NT, pl.lds, sd->rows, p, s);
}

extern "C" int dsv41_sampler_merge_run(const dsv41_sampler_merge_desc* d, void* stream) {
  if (!d) return fail(DSV41_E_INVALID, "sampler merge descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_sampler_merge_desc))
    return fail(DSV41_E_ABI, "dsv41_sampler_merge_desc size mismatch (rebuild the binding)");
  if (d->rows <= 0 || d->n_shards <= 0 || d->max_candidates <= 0)
    return fail(DSV41_E_INVALID, "sampler merge: rows, n_shards and max_candidates must be positive");
  if (!(d->top_k >= 1 && d->top_k <= KCAP)) return fail(DSV41_E_INVALID, "sampler merge: top_k must be in [1, 2048]");
  if (!(d->top_p > 0.0f && d->top_p <= 1.0f)) return fail(DSV41_E_INVALID, "top_p must be in (0, 1]");
  if (!(d->min_p >= 0.0f && d->min_p <= 1.0f)) return fail(DSV41_E_INVALID, "min_p must be in [0, 1]");
  if (!d->greedy && !d->uniforms) return fail(DSV41_E_INVALID, "sampling requires one uniform per row");
  if (!d->keys || !d->counts || !d->status || !d->out_ids || !d->out_status)
    return fail(DSV41_E_INVALID, "sampler merge: keys, counts, status, out_ids and out_status are required");
  const int64_t cap = (int64_t)d->n_shards * std::min<int64_t>(d->max_candidates, d->top_k);
  const size_t lds = merge_lds_bytes((size_t)cap, d->top_k);
  if (lds > LDS_LIMIT) return fail(DSV41_E_UNSUPPORTED, "sampler merge: n_shards * top_k exceeds the on-chip candidate buffer");
  Params p{};
  p.uniforms = d->uniforms;
  p.out_ids = d->out_ids;
  p.out_lp = d->out_logprob;
  p.out_kept = d->out_kept;
  p.out_status = d->out_status;
  p.log_min_p = d->min_p > 0.0f ? std::log((double)d->min_p) : -INFINITY;
  p.min_p = d->min_p;
  p.top_p = d->top_p;
  p.top_k = d->top_k;
  p.greedy = d->greedy ? 1 : 0;
  MergeIn in{d->keys, d->counts, d->status, d->n_shards, d->rows, d->max_candidates,
             std::min(d->max_candidates, d->top_k)};
  hipStream_t s = static_cast<hipStream_t>(stream);
  DSV41_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(merge_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_LIMIT));
  hipLaunchKernelGGL(merge_kernel, dim3(d->rows), dim3(TOPK_NT), lds, s, p, in);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}

// Checks a slice descriptor of a full-vocabulary draw and returns its Params.
// step: 0 = state, 1 = exact mass, 2 = draw
static int full_shard_params(const dsv41_sampler_full_shard_desc* d, int step, Plan* pl, Params* out) {
  if (!d) return fail(DSV41_E_INVALID, "sampler full shard descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_sampler_full_shard_desc))
    return fail(DSV41_E_ABI, "dsv41_sampler_full_shard_desc size mismatch (rebuild the binding)");
  const dsv41_sampler_desc* sd = d->sampler;
  if (!sd) return fail(DSV41_E_INVALID, "sampler full shard: the slice's sampler descriptor is NULL");
  int rc = plan(sd, pl, true);
  if (rc != DSV41_OK) return rc;
  if (pl->mode != MODE_FULL || sd->top_k != 0)
    return fail(DSV41_E_UNSUPPORTED, "vocabulary-sharded full-vocabulary draws take no top-k, top-p or min-p");
  if (sd->replay_ids) return fail(DSV41_E_UNSUPPORTED, "sampler full shard: replay_ids are not sharded");
  if (d->vocab_offset < 0 || d->vocab_size < d->vocab_offset + sd->vocab || d->vocab_size > MAX_VOCAB)
    return fail(DSV41_E_INVALID, "sampler shard: the slice must lie within a vocabulary of fewer than 2^21 ids");
  if (step > 0) {
    if (sd->greedy) return fail(DSV41_E_INVALID, "sampler full shard: greedy rows need no draw step (finish from the states)");
    if (d->n_shards <= 0 || d->shard_index < 0 || d->shard_index >= d->n_shards)
      return fail(DSV41_E_INVALID, "sampler full shard: shard_index must be in [0, n_shards)");
    if (!d->states) return fail(DSV41_E_INVALID, "sampler full shard: the gathered states are required");
  }
  if (step == 0 && !d->out_states) return fail(DSV41_E_INVALID, "sampler full shard: out_states is required");
  if (step == 1) {
    if (sd->exponentials)
      return fail(DSV41_E_INVALID, "sampler full shard: the exponential race needs no mass step");
    if (!d->out_masses) return fail(DSV41_E_INVALID, "sampler full shard: out_masses is required");
  }
  if (step == 2) {
    if (!d->out_picks) return fail(DSV41_E_INVALID, "sampler full shard: out_picks is required");
    if (!sd->exponentials && !sd->uniforms) return fail(DSV41_E_INVALID, "sampling requires one uniform per row");
    if (!sd->exponentials && !d->masses)
      return fail(DSV41_E_INVALID, "sampler full shard: an inverse-CDF draw needs the gathered masses");
  }
  Params p = make_params(sd, *pl, nullptr);
  p.greedy = 0;
  p.voff = (int)d->vocab_offset;
  p.vfull = (int)d->vocab_size;
  p.sh_states = d->states;
  p.sh_out_states = d->out_states;
  p.sh_out_picks = d->out_picks;
  p.sh_masses = d->masses;
  p.sh_out_masses = d->out_masses;
  p.n_shards = d->n_shards;
  p.shard_index = d->shard_index;
  p.nrows = sd->rows;
  *out = p;
  return DSV41_OK;
}

template <int DRAW>
static int launch_full(const Plan& pl, int rows, const Params& p, hipStream_t s) {
  if (pl.esize == 2) return pl.vec ? launch(full_kernel<uint16_t, 8, true, DRAW>, FULL_NT, pl.lds, rows, p, s)
                                   : launch(full_kernel<uint16_t, 8, false, DRAW>, FULL_NT, pl.lds, rows, p, s);
  return pl.vec ? launch(full_kernel<float, 8, true, DRAW>, FULL_NT, pl.lds, rows, p, s)
                : launch(full_kernel<float, 8, false, DRAW>, FULL_NT, pl.lds, rows, p, s);
}

extern "C" int dsv41_sampler_full_state_run(const dsv41_sampler_full_shard_desc* d, void* stream) {
  Plan pl;
  Params p;
  int rc = full_shard_params(d, 0, &pl, &p);
  if (rc != DSV41_OK) return rc;
  return launch_full<DRAW_STATE>(pl, d->sampler->rows, p, static_cast<hipStream_t>(stream));
}

extern "C" int dsv41_sampler_full_mass_run(const dsv41_sampler_full_shard_desc* d, void* stream) {
  Plan pl;
  Params p;
  int rc = full_shard_params(d, 1, &pl, &p);
  if (rc != DSV41_OK) return rc;
  return launch_full<DRAW_SHARD_MASS>(pl, d->sampler->rows, p, static_cast<hipStream_t>(stream));
}

extern "C" int dsv41_sampler_full_draw_run(const dsv41_sampler_full_shard_desc* d, void* stream) {
  Plan pl;
  Params p;
  int rc = full_shard_params(d, 2, &pl, &p);
  if (rc != DSV41_OK) return rc;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (d->sampler->exponentials) return launch_full<DRAW_SHARD_RACE>(pl, d->sampler->rows, p, s);
  return launch_full<DRAW_SHARD_CDF>(pl, d->sampler->rows, p, s);
}

extern "C" int dsv41_sampler_full_finish_run(const dsv41_sampler_full_finish_desc* d, void* stream) {
  if (!d) return fail(DSV41_E_INVALID, "sampler full finish descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_sampler_full_finish_desc))
    return fail(DSV41_E_ABI, "dsv41_sampler_full_finish_desc size mismatch (rebuild the binding)");
  if (d->rows <= 0 || d->n_shards <= 0)
    return fail(DSV41_E_INVALID, "sampler full finish: rows and n_shards must be positive");
  if (d->draw != DSV41_FULL_DRAW_CDF && d->draw != DSV41_FULL_DRAW_RACE && d->draw != DSV41_FULL_DRAW_GREEDY)
    return fail(DSV41_E_INVALID, "sampler full finish: draw must be DSV41_FULL_DRAW_CDF, _RACE or _GREEDY");
  if (!d->states || (d->draw != DSV41_FULL_DRAW_GREEDY && !d->picks))
    return fail(DSV41_E_INVALID, "sampler full finish: states (and picks, unless greedy) are required");
  if (d->draw == DSV41_FULL_DRAW_CDF && !d->uniforms) return fail(DSV41_E_INVALID, "sampling requires one uniform per row");
  if (!d->out_ids || !d->out_status) return fail(DSV41_E_INVALID, "out_ids and out_status are required");
  hipLaunchKernelGGL(full_finish_kernel, dim3((d->rows + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream),
                     *d);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}
