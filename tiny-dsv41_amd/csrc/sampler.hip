// sampler.hip — row sampler for gfx950: penalties over per-row history, temperature,
// min-p / top-k / top-p, greedy or inverse-CDF draw against caller uniforms, and the
// drawn token's log-prob under the processed distribution.
//
// Replaces the sampling step of generate_group (dsv41_train/rl/rollout.py:144-150:
// log_softmax(logits.float() / T), finite check, draw, behaviour log-prob) for a
// [rows, vocab] batch, with the vLLM SamplingParams knobs of
// rollout_manager/backends/vllm_actor.py:178-185 applied in vLLM v1's order.
//
// One workgroup per row streams the row from HBM exactly once:
//   FULL    (no truncation): per-chunk (max, sum exp) in LDS, float inverse CDF over
//           chunk sums, then one 64*G-element chunk is re-read to place the draw.
//   TOPK    (1 <= top_k <= 4096): elements above a running threshold (top-k of what
//           has been seen, and the min-p bound from the running max) go to an LDS
//           candidate buffer; after the pass the buffer is sorted and every decision
//           (min-p, top-k, top-p, draw) is an exact scan over it.
//   GENERIC (anything else that truncates): z is written to a workspace row and the
//           same decisions are made by exact radix selection over it.
// Selection arithmetic is exact (fp32 compares, fp64 differences of fp32 values,
// 64-bit fixed-point masses), so kept sets and ids do not depend on reduction order.
// This file is compiled with -ffp-contract=off: each operation rounds as written.

#include <math.h>
#include <string.h>

#include <mutex>

#include "common.h"

namespace dsv41 {
namespace sampler {

constexpr int MODE_FULL = 0;
constexpr int MODE_TOPK = 1;
constexpr int MODE_GENERIC = 2;

constexpr int NT = 1024;          // threads per workgroup (16 waves)
constexpr int NW = NT / 64;
constexpr int TOPK_G = 4;         // elements per thread per tile in TOPK mode
constexpr int TOPK_TILE = NT * TOPK_G;
constexpr int TOPK_CAP = 8192;    // candidate buffer entries (u64 keys)
constexpr int KCAP = TOPK_CAP - TOPK_TILE;  // largest top_k on the one-pass path
constexpr int MAX_VOCAB = 1 << 21;          // 2^21 * 2^43 < 2^64: mass sums cannot wrap
constexpr size_t LDS_LIMIT = 160 * 1024;

constexpr float NEG_INF = -__builtin_huge_valf();
constexpr float LOG2E = 1.4426950408889634f;

constexpr int ST_NONFINITE = DSV41_STATUS_NONFINITE;
constexpr int ST_BAD_HISTORY = DSV41_STATUS_BAD_HISTORY;
constexpr int ST_BAD_UNIFORM = DSV41_STATUS_BAD_UNIFORM;

struct Params {
  const void* logits;
  int64_t lstride;
  const int64_t* hist;
  int64_t hstride;
  const int32_t* hlens;
  const float* uniforms;
  int64_t* out_ids;
  float* out_lp;
  int32_t* out_kept;
  int32_t* out_status;
  float* zbuf;
  double log_min_p;
  float T, rT, rp, pres, freq, top_p, min_p;
  int V, hlen, top_k, greedy, has_pen, unit_T, fast_div, ucap, words;
};

// Per-workgroup scalars and reduction scratch, at the start of dynamic LDS.
struct Misc {
  double rd[NW];
  uint64_t ru[NW];
  float rf[NW];
  float wmax[NW];
  int ri[NW];
  uint64_t bu[4];
  double bd[4];
  float bf[4];
  int bi[4];
  int status;
  int count;
  int U;
  float tau;
  uint64_t tau_key;
};

struct Layout {
  size_t misc, bitmap, wrank, cnt, penx, hist256, mode0, total;
};

__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~(size_t)15; }

template <int G>
__host__ __device__ inline int n_chunks(int V) {
  return (V + 64 * G - 1) / (64 * G);
}

// LDS layout; must agree between the launch (host) and the kernel (device).
template <int MODE, int G>
__host__ __device__ inline Layout make_layout(int V, int words, int ucap) {
  Layout l;
  size_t off = 0;
  l.misc = off;
  off = align16(off + sizeof(Misc));
  l.bitmap = off;
  off += 4 * (size_t)words;
  l.wrank = off;
  off += 4 * (size_t)words;
  l.cnt = off;
  off += 4 * (size_t)ucap;
  l.penx = off;
  off = align16(off + 4 * (size_t)ucap);
  l.hist256 = off;
  off += 256 * 8;
  l.mode0 = off;
  if (MODE == MODE_FULL) off += 8 * (size_t)n_chunks<G>(V);
  if (MODE == MODE_TOPK) off += 8 * (size_t)TOPK_CAP;
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

__device__ __forceinline__ uint64_t mass_of(float z, float zmax) {
  return (uint64_t)(exp_det((double)z - (double)zmax) * 8796093022208.0);  // 2^43
}

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
  x = x - p.pres;
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
__device__ __forceinline__ float block_max(float v, Misc* m) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_max(v);
  if (lane == 0) m->rf[wid] = v;
  __syncthreads();
  float r = m->rf[0];
  for (int i = 1; i < NW; ++i) r = fmaxf(r, m->rf[i]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ int block_sum_i(int v, Misc* m) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum_i(v);
  if (lane == 0) m->ri[wid] = v;
  __syncthreads();
  int r = 0;
  for (int i = 0; i < NW; ++i) r += m->ri[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ int block_min_i(int v, Misc* m) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_min_i(v);
  if (lane == 0) m->ri[wid] = v;
  __syncthreads();
  int r = m->ri[0];
  for (int i = 1; i < NW; ++i) r = min(r, m->ri[i]);
  __syncthreads();
  return r;
}
__device__ __forceinline__ uint64_t block_sum_u64(uint64_t v, Misc* m) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum_u64(v);
  if (lane == 0) m->ru[wid] = v;
  __syncthreads();
  uint64_t r = 0;
  for (int i = 0; i < NW; ++i) r += m->ru[i];
  __syncthreads();
  return r;
}
__device__ __forceinline__ double block_sum_d(double v, Misc* m) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_sum_d(v);
  if (lane == 0) m->rd[wid] = v;
  __syncthreads();
  double r = 0.0;
  for (int i = 0; i < NW; ++i) r += m->rd[i];
  __syncthreads();
  return r;
}

// In-place inclusive prefix sum of a[0..n), n <= 4 * NT.
__device__ void block_incl_scan_u64(uint64_t* a, int n, Misc* m) {
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

// Descending bitonic sort of a[0..n) (u64 keys), padding to a power of two with 0.
__device__ void bitonic_sort_desc(uint64_t* a, int n) {
  const int tid = threadIdx.x;
  int P = 2;
  while (P < n) P <<= 1;
  for (int i = n + tid; i < P; i += NT) a[i] = 0;
  __syncthreads();
  for (int k = 2; k <= P; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < (P >> 1); i += NT) {
        const int lo = ((i & ~(j - 1)) << 1) | (i & (j - 1));
        const int hi = lo + j;
        const bool desc = (lo & k) == 0;
        const uint64_t x = a[lo], y = a[hi];
        if ((x < y) == desc) {
          a[lo] = y;
          a[hi] = x;
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
template <bool DESC, int NBITS, class Visit>
__device__ uint64_t radix_select(Visit visit, uint64_t target, uint64_t* hist, Misc* m,
                                 bool* found) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  uint64_t prefix = 0, mask = 0;
  bool ok = true;
  for (int shift = ((NBITS + 7) / 8 - 1) * 8; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += NT) hist[i] = 0;
    __syncthreads();
    visit([&](uint64_t key, uint64_t w) {
      if (w != 0 && (key & mask) == prefix) atomicAdd((unsigned long long*)&hist[(key >> shift) & 255], (unsigned long long)w);
    });
    __syncthreads();
    if (wid == 0) {
      // lane l owns 4 bins in traversal order
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
      const bool mine = before < target && target <= incl;
      if (mine) {
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

// ------------------------------------------------------------ history tables
// bitmap[w] bit b set <=> token 32w+b occurs in the row's history;
// wrank[w] = number of set bits before word w (slot of the word's first token);
// cnt[slot] = occurrences.  Returns the number of distinct tokens.
__device__ int build_history(const Params& p, int row, uint32_t* bitmap, uint32_t* wrank,
                             uint32_t* cnt, Misc* m) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int W = p.words;
  for (int i = tid; i < W; i += NT) bitmap[i] = 0;
  for (int i = tid; i < p.ucap; i += NT) cnt[i] = 0;
  __syncthreads();
  int hl = p.hlens ? p.hlens[row] : p.hlen;
  hl = max(0, min(hl, (int)p.hstride));
  const int64_t* h = p.hist + (int64_t)row * p.hstride;
  int bad = 0;
  for (int j = tid; j < hl; j += NT) {
    const int64_t id = h[j];
    if (id >= 0 && id < p.V)
      atomicOr(&bitmap[id >> 5], 1u << (id & 31));
    else if (id >= p.V)
      bad = 1;
  }
  if (bad) atomicOr(&m->status, ST_BAD_HISTORY);
  __syncthreads();
  // exclusive prefix popcount over words
  const int per = (W + NT - 1) / NT;
  const int b = tid * per, e = min(b + per, W);
  int s = 0;
  for (int i = b; i < e; ++i) s += __popc(bitmap[i]);
  const int incl = wave_incl_scan_i(s, lane);
  if (lane == 63) m->ri[wid] = incl;
  __syncthreads();
  int off = 0;
  for (int i = 0; i < wid; ++i) off += m->ri[i];
  int run = off + incl - s;
  for (int i = b; i < e; ++i) {
    wrank[i] = (uint32_t)run;
    run += __popc(bitmap[i]);
  }
  int U = 0;
  for (int i = 0; i < NW; ++i) U += m->ri[i];
  __syncthreads();
  for (int j = tid; j < hl; j += NT) {
    const int64_t id = h[j];
    if (id >= 0 && id < p.V) {
      const uint32_t w = (uint32_t)(id >> 5), bit = (uint32_t)(id & 31);
      const uint32_t slot = wrank[w] + __popc(bitmap[w] & ((1u << bit) - 1u));
      atomicAdd(&cnt[slot], 1u);
    }
  }
  __syncthreads();
  return U;
}

// Token id of history slot s (the s-th set bit of the bitmap).
__device__ int slot_token(int s, const uint32_t* bitmap, const uint32_t* wrank, int W) {
  int lo = 0, hi = W - 1;  // largest w with wrank[w] <= s
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((int)wrank[mid] <= s) lo = mid;
    else hi = mid - 1;
  }
  uint32_t word = bitmap[lo];
  for (int k = s - (int)wrank[lo]; k > 0; --k) word &= word - 1u;
  return lo * 32 + (__ffs(word) - 1);
}

// Processed logit of history slot s from its captured raw logit penx[s].
__device__ __forceinline__ float slot_z(int s, const uint32_t* cnt, const float* penx,
                                        const Params& p) {
  const float x = penalize(penx[s], cnt[s], p);
  return x / p.T;
}

// ------------------------------------------------------------ streaming
template <typename TIn, int G>
struct Raw {
  static constexpr int WORDS = G * (int)sizeof(TIn) / 4;
  uint32_t w[WORDS];
};

template <typename TIn, int G, bool VEC>
__device__ __forceinline__ void load_raw(const TIn* row, int base, int V, Raw<TIn, G>& r) {
  constexpr int WORDS = Raw<TIn, G>::WORDS;
  if (VEC && base + G <= V) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(row + base);
    if constexpr (WORDS == 4) {
      const uint4 v = *reinterpret_cast<const uint4*>(src);
      r.w[0] = v.x;
      r.w[1] = v.y;
      r.w[2] = v.z;
      r.w[3] = v.w;
    } else if constexpr (WORDS == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(src);
      r.w[0] = v.x;
      r.w[1] = v.y;
    } else {
#pragma unroll
      for (int i = 0; i < WORDS; ++i) r.w[i] = src[i];
    }
  } else {
    // scalar path: unaligned rows and the ragged tail
#pragma unroll
    for (int i = 0; i < WORDS; ++i) r.w[i] = 0;
    if constexpr (sizeof(TIn) == 4) {
#pragma unroll
      for (int j = 0; j < G; ++j)
        if (base + j < V) r.w[j] = reinterpret_cast<const uint32_t*>(row)[base + j];
    } else {
#pragma unroll
      for (int j = 0; j < G; ++j)
        if (base + j < V) {
          const uint32_t h = reinterpret_cast<const uint16_t*>(row)[base + j];
          r.w[j >> 1] |= (j & 1) ? (h << 16) : h;
        }
    }
  }
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

// Turns G raw logits at [base, base+G) into processed z (penalized tokens and the
// tail become -inf; penalized raw logits are captured into penx[slot]).
template <int G, bool CAPTURE = true>
__device__ __forceinline__ void process_group(float (&x)[G], int base, const Params& p,
                                              const uint32_t* bitmap, const uint32_t* wrank,
                                              float* penx, float (&z)[G], int& bad) {
  uint32_t pen = 0;
  if (p.has_pen && base < p.V) {
    const uint32_t word = bitmap[base >> 5];
    const uint32_t sh = (uint32_t)base & 31u;
    pen = (word >> sh) & ((1u << G) - 1u);
    if (CAPTURE && pen) {
      const uint32_t r0 = wrank[base >> 5] + __popc(word & ((1u << sh) - 1u));
#pragma unroll
      for (int j = 0; j < G; ++j)
        if ((pen >> j) & 1u) penx[r0 + __popc(pen & ((1u << j) - 1u))] = x[j];
    }
  }
  // 2^-100 <= |x| < 2^100: three-operation division is IEEE-exact there (checked
  // exhaustively on the host for the oracle); outside it, IEEE division.
  uint32_t lo = 0xFFFFFFFFu, hi = 0;
#pragma unroll
  for (int j = 0; j < G; ++j) {
    const uint32_t a = __float_as_uint(x[j]) & 0x7FFFFFFFu;
    lo = min(lo, a);
    hi = max(hi, a);
  }
  const bool fast = p.fast_div && lo >= 0x0D800000u && hi < 0x71800000u;
  if (fast) {
    if (p.unit_T) {
#pragma unroll
      for (int j = 0; j < G; ++j) z[j] = x[j];
    } else {
#pragma unroll
      for (int j = 0; j < G; ++j) {
        const float q = x[j] * p.rT;
        const float e = __builtin_fmaf(-q, p.T, x[j]);
        z[j] = __builtin_fmaf(e, p.rT, q);
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < G; ++j) {
      z[j] = x[j] / p.T;
      if (base + j < p.V && !((pen >> j) & 1u) && !isfinite(z[j])) bad = 1;
    }
  }
#pragma unroll
  for (int j = 0; j < G; ++j)
    if (base + j >= p.V || ((pen >> j) & 1u)) z[j] = NEG_INF;
}

template <typename TIn>
__device__ __forceinline__ const TIn* row_ptr(const Params& p, int row) {
  return reinterpret_cast<const TIn*>(p.logits) + (int64_t)row * p.lstride;
}

__device__ __forceinline__ void write_result(const Params& p, int row, Misc* m, int64_t id,
                                             float lp, int kept) {
  const int st = m->status;
  if (st & ST_NONFINITE) {
    p.out_ids[row] = -1;
    p.out_lp[row] = __builtin_nanf("");
    if (p.out_kept) p.out_kept[row] = 0;
  } else {
    p.out_ids[row] = id;
    p.out_lp[row] = lp;
    if (p.out_kept) p.out_kept[row] = kept;
  }
  p.out_status[row] = st;
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

// ====================================================================== FULL
// No truncation: kept set = whole vocabulary.  Chunk c = [c*64G, (c+1)*64G) is one
// wave's span of one tile; its (max, sum exp(z - max)) go to LDS.
template <typename TIn, int G, bool VEC>
__global__ __launch_bounds__(NT) void full_kernel(Params p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const Layout L = make_layout<MODE_FULL, G>(p.V, p.words, p.ucap);
  Misc* m = reinterpret_cast<Misc*>(smem + L.misc);
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(smem + L.bitmap);
  uint32_t* wrank = reinterpret_cast<uint32_t*>(smem + L.wrank);
  uint32_t* cnt = reinterpret_cast<uint32_t*>(smem + L.cnt);
  float* penx = reinterpret_cast<float*>(smem + L.penx);
  const int NC = n_chunks<G>(p.V);
  float* cm = reinterpret_cast<float*>(smem + L.mode0);
  float* cs = cm + NC;

  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) m->status = 0;
  __syncthreads();
  int U = 0;
  if (p.has_pen) U = build_history(p, row, bitmap, wrank, cnt, m);
  const TIn* src = row_ptr<TIn>(p, row);
  constexpr int TILE = NT * G;
  const int ntiles = (p.V + TILE - 1) / TILE;
  int bad = 0;

  Raw<TIn, G> r0, r1;
  load_raw<TIn, G, VEC>(src, tid * G, p.V, r0);
  if (ntiles > 1) load_raw<TIn, G, VEC>(src, TILE + tid * G, p.V, r1);
  for (int t = 0; t < ntiles; ++t) {
    Raw<TIn, G> r2;
    if (t + 2 < ntiles) load_raw<TIn, G, VEC>(src, (t + 2) * TILE + tid * G, p.V, r2);
    const int base = t * TILE + tid * G;
    float x[G], z[G];
    unpack(r0, x);
    process_group<G>(x, base, p, bitmap, wrank, penx, z, bad);
    float mx = z[0];
#pragma unroll
    for (int j = 1; j < G; ++j) mx = fmaxf(mx, z[j]);
    mx = wave_max(mx);
    float s = 0.0f;
    if (mx > NEG_INF) {
      const float mb = mx * LOG2E;
#pragma unroll
      for (int j = 0; j < G; ++j) s += exp2f(__builtin_fmaf(z[j], LOG2E, -mb));
    }
    s = wave_sum(s);
    const int c = t * NW + wid;
    if (lane == 0 && c < NC) {
      cm[c] = mx;
      cs[c] = s;
    }
    r0 = r1;
    r1 = r2;
  }
  if (bad) atomicOr(&m->status, ST_NONFINITE);
  __syncthreads();

  // penalized tokens: exact z, written back over the captured raw logits
  float pmax = NEG_INF;
  for (int s = tid; s < U; s += NT) {
    const float z = slot_z(s, cnt, penx, p);
    if (!isfinite(z)) atomicOr(&m->status, ST_NONFINITE);
    penx[s] = z;
    pmax = fmaxf(pmax, z);
  }
  float cmax = NEG_INF;
  for (int c = tid; c < NC; c += NT) cmax = fmaxf(cmax, cm[c]);
  const float M = block_max(fmaxf(pmax, cmax), m);  // also orders the penx writes

  // rescale chunk sums to the row maximum, then add the penalized tokens
  for (int c = tid; c < NC; c += NT) cs[c] = cm[c] > NEG_INF ? cs[c] * exp2f((cm[c] - M) * LOG2E) : 0.0f;
  __syncthreads();
  for (int s = tid; s < U; s += NT) {
    const int tok = slot_token(s, bitmap, wrank, p.words);
    atomicAdd(&cs[tok / (64 * G)], exp2f((penx[s] - M) * LOG2E));
  }
  __syncthreads();

  // total mass and chunk prefix (wave 0, fp64)
  const float u = row_uniform(p, row, m);
  if (wid == 0) {
    const int per = (NC + 63) / 64;
    const int b = lane * per, e = min(b + per, NC);
    double s = 0.0;
    for (int c = b; c < e; ++c) s += (double)cs[c];
    const double incl = wave_incl_scan_d(s, lane);
    const double S = __shfl(incl, 63);
    const double t = (double)u * S;
    double before = incl - s;
    // chunk holding t: the one whose [before, before + cs) contains t
    int cstar = -1;
    double cbefore = 0.0;
    if (before <= t && t < incl) {
      int lastpos = -1;
      for (int c = b; c < e; ++c) {
        if (cs[c] > 0.0f) lastpos = c;
        if (t < before + (double)cs[c]) {
          cstar = c;
          cbefore = before;
          break;
        }
        before += (double)cs[c];
      }
      if (cstar < 0 && lastpos >= 0) {  // rounding: last positive chunk, last element
        cstar = lastpos;
        cbefore = t + 1.0;
      }
    }
    // rounding fallback: the last chunk with positive mass
    unsigned long long hit = __ballot(cstar >= 0);
    if (hit == 0) {
      int last = -1;
      for (int c = b; c < e; ++c)
        if (cs[c] > 0.0f) last = c;
      int lastmax = last;
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) lastmax = max(lastmax, __shfl_xor(lastmax, o));
      if (lane == 0) {
        m->bi[0] = lastmax;
        m->bd[0] = -1.0;  // take the last positive element of that chunk
      }
    } else {
      const int src_lane = __ffsll((long long)hit) - 1;
      cstar = __shfl(cstar, src_lane);
      cbefore = __shfl(cbefore, src_lane);
      if (lane == 0) {
        m->bi[0] = cstar;
        m->bd[0] = t - cbefore;
      }
    }
    if (lane == 0) m->bd[1] = S;
  }
  // first chunk whose maximum is the row maximum (for greedy)
  int cfirst = NC;
  for (int c = tid; c < NC; c += NT)
    if (cm[c] == M) cfirst = min(cfirst, c);
  int pfirst = 0x7FFFFFFF;
  for (int s = tid; s < U; s += NT)
    if (penx[s] == M) pfirst = min(pfirst, slot_token(s, bitmap, wrank, p.words));
  cfirst = block_min_i(cfirst, m);
  pfirst = block_min_i(pfirst, m);  // barriers: m->bi/bd visible after this

  if (wid == 0) {
    const double S = m->bd[1];
    int64_t tok = 0;
    float ztok = M;
    if (p.greedy) {
      int best = pfirst;
      if (cfirst < NC) {
        const int base = cfirst * 64 * G + lane * G;
        Raw<TIn, G> r;
        load_raw<TIn, G, VEC>(src, base, p.V, r);
        float x[G], z[G];
        unpack(r, x);
        int dummy = 0;
        process_group<G, false>(x, base, p, bitmap, wrank, penx, z, dummy);
        int first = 0x7FFFFFFF;
#pragma unroll
        for (int j = G - 1; j >= 0; --j)
          if (z[j] == M) first = base + j;
        first = wave_min_i(first);
        best = min(best, first);
      }
      tok = best;
      ztok = M;
    } else if (m->bi[0] < 0) {
      // no chunk carries mass: only rows without a finite maximum (flagged non-finite)
      tok = 0;
      ztok = M;
    } else {
      const int cstar = m->bi[0];
      const double need = m->bd[0];
      const int base = cstar * 64 * G + lane * G;
      Raw<TIn, G> r;
      load_raw<TIn, G, VEC>(src, base, p.V, r);
      float x[G], z[G], e[G];
      unpack(r, x);
      int dummy = 0;
      process_group<G, false>(x, base, p, bitmap, wrank, penx, z, dummy);
      // restore penalized elements of this chunk from their exact z
      if (p.has_pen) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
          const int v = base + j;
          if (v < p.V) {
            const uint32_t word = bitmap[v >> 5];
            if ((word >> (v & 31)) & 1u) z[j] = penx[wrank[v >> 5] + __popc(word & ((1u << (v & 31)) - 1u))];
          }
        }
      }
      double ls = 0.0;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        e[j] = exp2f((z[j] - M) * LOG2E);
        ls += (double)e[j];
      }
      const double incl = wave_incl_scan_d(ls, lane);
      double acc = incl - ls;
      int pick = -1;
      int lastpos = -1;
#pragma unroll
      for (int j = 0; j < G; ++j) {
        if (e[j] > 0.0f) lastpos = base + j;
        if (pick < 0 && need >= 0.0 && need < acc + (double)e[j] && e[j] > 0.0f) pick = base + j;
        acc += (double)e[j];
      }
      const unsigned long long hit = __ballot(pick >= 0);
      int chosen;
      if (hit) {
        chosen = __shfl(pick, __ffsll((long long)hit) - 1);
      } else {
        int lp = lastpos;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) lp = max(lp, __shfl_xor(lp, o));
        chosen = lp;
      }
      // z of the chosen element
      float zc = NEG_INF;
#pragma unroll
      for (int j = 0; j < G; ++j)
        if (base + j == chosen) zc = z[j];
      zc = wave_max(zc);
      tok = chosen;
      ztok = zc;
    }
    if (lane == 0) {
      const float lp = (float)(((double)ztok - (double)M) - log(S));
      write_result(p, row, m, tok, lp, p.V);
    }
  }
}

// ====================================================================== TOPK
// One pass: elements with z above the running threshold go to an LDS buffer of
// ckeys.  Before each tile the buffer is compacted if it could overflow: sorted,
// cut to top_k and to the min-p bound of the running maximum.
__device__ void topk_compact(uint64_t* cand, Misc* m, const Params& p, float mrun) {
  const int tid = threadIdx.x;
  const int n = m->count;
  bitonic_sort_desc(cand, n);
  int el = 0;
  if (p.min_p > 0.0f && mrun > NEG_INF) {
    for (int i = tid; i < n; i += NT) el += minp_ok(ckey_z(cand[i]), mrun, p) ? 1 : 0;
    el = block_sum_i(el, m);
  } else {
    el = n;
  }
  const int keep = min(el, p.top_k);
  if (tid == 0) {
    if (keep == p.top_k && keep > 0) {
      m->tau = ckey_z(cand[keep - 1]);
      m->tau_key = cand[keep - 1];
    }
    m->count = keep;
  }
  __syncthreads();
}

__device__ __forceinline__ float minp_bound(float mrun, const Params& p) {
  if (!(p.min_p > 0.0f) || !(mrun > NEG_INF)) return NEG_INF;
  // conservative fp32 lower bound of mrun + log(min_p)
  const double d = (double)mrun + p.log_min_p;
  const double slack = 1e-6 * (fabs((double)mrun) + fabs(p.log_min_p) + 1.0);
  return (float)(d - slack);
}

template <typename TIn, bool VEC>
__global__ __launch_bounds__(NT) void topk_kernel(Params p) {
  constexpr int G = TOPK_G;
  extern __shared__ __align__(16) unsigned char smem[];
  const Layout L = make_layout<MODE_TOPK, G>(p.V, p.words, p.ucap);
  Misc* m = reinterpret_cast<Misc*>(smem + L.misc);
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(smem + L.bitmap);
  uint32_t* wrank = reinterpret_cast<uint32_t*>(smem + L.wrank);
  uint32_t* cnt = reinterpret_cast<uint32_t*>(smem + L.cnt);
  float* penx = reinterpret_cast<float*>(smem + L.penx);
  uint64_t* hist = reinterpret_cast<uint64_t*>(smem + L.hist256);
  uint64_t* cand = reinterpret_cast<uint64_t*>(smem + L.mode0);

  const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  if (tid == 0) {
    m->status = 0;
    m->count = 0;
    m->tau = NEG_INF;
    m->tau_key = 0;
  }
  if (tid < NW) m->wmax[tid] = NEG_INF;
  __syncthreads();
  int U = 0;
  if (p.has_pen) U = build_history(p, row, bitmap, wrank, cnt, m);
  const TIn* src = row_ptr<TIn>(p, row);
  constexpr int TILE = TOPK_TILE;
  const int ntiles = (p.V + TILE - 1) / TILE;
  int bad = 0;

  Raw<TIn, G> r0, r1, r2;
  load_raw<TIn, G, VEC>(src, tid * G, p.V, r0);
  if (ntiles > 1) load_raw<TIn, G, VEC>(src, TILE + tid * G, p.V, r1);
  if (ntiles > 2) load_raw<TIn, G, VEC>(src, 2 * TILE + tid * G, p.V, r2);
  for (int t = 0; t < ntiles; ++t) {
    Raw<TIn, G> r3;
    if (t + 3 < ntiles) load_raw<TIn, G, VEC>(src, (t + 3) * TILE + tid * G, p.V, r3);
    const int base = t * TILE + tid * G;
    float x[G], z[G];
    unpack(r0, x);
    process_group<G>(x, base, p, bitmap, wrank, penx, z, bad);
    float mx = z[0];
#pragma unroll
    for (int j = 1; j < G; ++j) mx = fmaxf(mx, z[j]);
    mx = wave_max(mx);
    if (lane == 0) m->wmax[wid] = fmaxf(m->wmax[wid], mx);
    __syncthreads();
    float mrun = m->wmax[0];
    for (int i = 1; i < NW; ++i) mrun = fmaxf(mrun, m->wmax[i]);
    const int cnow = m->count;
    __syncthreads();  // every wave has read the count before any inserts
    if (cnow + TILE > TOPK_CAP) topk_compact(cand, m, p, mrun);
    const float tau = m->tau;
    const float tmp = minp_bound(mrun, p);
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const bool pred = z[j] > tau && z[j] >= tmp;
      const unsigned long long bal = __ballot(pred);
      if (bal) {
        const uint32_t before = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        int pos0 = 0;
        if (lane == 0) pos0 = atomicAdd(&m->count, (int)__popcll(bal));
        pos0 = __shfl(pos0, 0);
        if (pred) cand[pos0 + (int)before] = ckey(z[j], (uint32_t)(base + j));
      }
    }
    r0 = r1;
    r1 = r2;
    r2 = r3;
  }
  if (bad) atomicOr(&m->status, ST_NONFINITE);
  __syncthreads();

  // penalized tokens (arbitrary indices: compare full keys against the k-th key)
  if (U > 0) {
    float mrun = m->wmax[0];
    for (int i = 1; i < NW; ++i) mrun = fmaxf(mrun, m->wmax[i]);
    float pm = NEG_INF;
    for (int s = tid; s < U; s += NT) {
      const float z = slot_z(s, cnt, penx, p);
      if (!isfinite(z)) atomicOr(&m->status, ST_NONFINITE);
      penx[s] = z;
      pm = fmaxf(pm, z);
    }
    pm = block_max(pm, m);
    mrun = fmaxf(mrun, pm);
    for (int s0 = 0; s0 < U; s0 += NT) {
      const int cnow = m->count;
      __syncthreads();
      if (cnow + NT > TOPK_CAP) topk_compact(cand, m, p, mrun);
      const uint64_t tk = m->tau_key;
      const float tmp = minp_bound(mrun, p);
      const int s = s0 + tid;
      bool pred = false;
      uint64_t key = 0;
      if (s < U) {
        const float z = penx[s];
        key = ckey(z, (uint32_t)slot_token(s, bitmap, wrank, p.words));
        pred = key > tk && z >= tmp && z > NEG_INF;
      }
      const unsigned long long bal = __ballot(pred);
      if (bal) {
        const uint32_t before = __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        int pos0 = 0;
        if (lane == 0) pos0 = atomicAdd(&m->count, (int)__popcll(bal));
        pos0 = __shfl(pos0, 0);
        if (pred) cand[pos0 + (int)before] = key;
      }
      __syncthreads();
    }
  }

  // final selection over the candidates
  const int n = m->count;
  bitonic_sort_desc(cand, n);
  const float u = row_uniform(p, row, m);
  const float zmax = ckey_z(cand[0]);
  int el = 0;
  for (int i = tid; i < n; i += NT) el += minp_ok(ckey_z(cand[i]), zmax, p) ? 1 : 0;
  el = block_sum_i(el, m);
  const int K = min(p.top_k, el);
  if (K == 0) {  // only possible for rows without a finite maximum
    if (tid == 0) {
      m->status |= ST_NONFINITE;
      write_result(p, row, m, -1, 0.0f, 0);
    }
    return;
  }
  uint64_t* q = cand + TOPK_CAP / 2;  // K <= KCAP = TOPK_CAP / 2 entries, beyond the prefix
  for (int i = tid; i < K; i += NT) q[i] = mass_of(ckey_z(cand[i]), zmax);
  __syncthreads();
  int n_keep = K;
  uint64_t S;
  if (p.top_p < 1.0f) {
    block_incl_scan_u64(q, K, m);
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
    S = block_sum_u64(s, m);
  }
  double es = 0.0;
  for (int i = tid; i < n_keep; i += NT) es += exp_det((double)ckey_z(cand[i]) - (double)zmax);
  const double esum = block_sum_d(es, m);

  int64_t tok;
  float ztok;
  if (p.greedy) {
    tok = ckey_idx(cand[0]);
    ztok = zmax;
  } else {
    const uint64_t t = draw_target(u, S);
    bool found = false;
    const uint64_t idx = radix_select<false, 24>(
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

// ====================================================================== GENERIC
template <typename TIn, int G, bool VEC>
__global__ __launch_bounds__(NT) void generic_kernel(Params p) {
  extern __shared__ __align__(16) unsigned char smem[];
  const Layout L = make_layout<MODE_GENERIC, G>(p.V, p.words, p.ucap);
  Misc* m = reinterpret_cast<Misc*>(smem + L.misc);
  uint32_t* bitmap = reinterpret_cast<uint32_t*>(smem + L.bitmap);
  uint32_t* wrank = reinterpret_cast<uint32_t*>(smem + L.wrank);
  uint32_t* cnt = reinterpret_cast<uint32_t*>(smem + L.cnt);
  float* penx = reinterpret_cast<float*>(smem + L.penx);
  uint64_t* hist = reinterpret_cast<uint64_t*>(smem + L.hist256);

  const int row = blockIdx.x, tid = threadIdx.x;
  if (tid == 0) m->status = 0;
  __syncthreads();
  int U = 0;
  if (p.has_pen) U = build_history(p, row, bitmap, wrank, cnt, m);
  const TIn* src = row_ptr<TIn>(p, row);
  float* zr = p.zbuf + (int64_t)row * p.V;
  constexpr int TILE = NT * G;
  const int ntiles = (p.V + TILE - 1) / TILE;
  int bad = 0;
  for (int t = 0; t < ntiles; ++t) {
    const int base = t * TILE + tid * G;
    Raw<TIn, G> r;
    load_raw<TIn, G, VEC>(src, base, p.V, r);
    float x[G], z[G];
    unpack(r, x);
    process_group<G>(x, base, p, bitmap, wrank, penx, z, bad);
#pragma unroll
    for (int j = 0; j < G; ++j)
      if (base + j < p.V) zr[base + j] = z[j];
  }
  if (bad) atomicOr(&m->status, ST_NONFINITE);
  __syncthreads();
  for (int s = tid; s < U; s += NT) {
    const float z = slot_z(s, cnt, penx, p);
    if (!isfinite(z)) atomicOr(&m->status, ST_NONFINITE);
    zr[slot_token(s, bitmap, wrank, p.words)] = z;
  }
  __threadfence_block();
  __syncthreads();

  const int V = p.V;
  // row maximum and its first index
  float bm = NEG_INF;
  int bi = 0x7FFFFFFF;
  for (int i = tid; i < V; i += NT) {
    const float z = zr[i];
    if (z > bm) {
      bm = z;
      bi = i;
    }
  }
  const float zmax = block_max(bm, m);
  int am = block_min_i(bm == zmax ? bi : 0x7FFFFFFF, m);
  if (am < 0 || am >= V) am = 0;  // no finite maximum: the row is flagged non-finite
  const float u = row_uniform(p, row, m);

  int el = 0;
  for (int i = tid; i < V; i += NT) el += minp_ok(zr[i], zmax, p) ? 1 : 0;
  el = block_sum_i(el, m);
  const int K = (p.top_k > 0 && p.top_k < el) ? p.top_k : el;
  bool found = false;
  uint64_t B1 = 0;
  if (K < el) {
    B1 = radix_select<true, 64>(
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
    s1 = block_sum_u64(s1, m);
    const uint64_t thr = top_p_threshold(p.top_p, s1);
    B = radix_select<true, 64>(
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
  nk = block_sum_i(nk, m);
  sk = block_sum_u64(sk, m);
  const double esum = block_sum_d(es, m);
  int64_t tok = am;
  if (!p.greedy) {
    const uint64_t t = draw_target(u, sk);
    const uint64_t idx = radix_select<false, 24>(
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
}

// ====================================================================== host
template <class K>
int launch(K kernel, size_t lds, int rows, const Params& prm, hipStream_t stream) {
  DSV41_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  hipLaunchKernelGGL(kernel, dim3(rows), dim3(NT), lds, stream, prm);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}

struct Plan {
  int mode;
  int esize;
  bool vec;
  bool has_pen;
  int words, ucap;
  size_t lds;
  size_t workspace;
};

int plan(const dsv41_sampler_desc* d, Plan* pl) {
  if (!d) return fail(DSV41_E_INVALID, "sampler descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_sampler_desc))
    return fail(DSV41_E_ABI, "dsv41_sampler_desc size mismatch (rebuild the binding)");
  if (d->rows <= 0 || d->vocab <= 0)
    return fail(DSV41_E_INVALID, "logits must have shape [rows, vocabulary_size] with both nonzero");
  if (d->vocab > MAX_VOCAB) return fail(DSV41_E_UNSUPPORTED, "vocabulary_size above 2^21 is not supported");
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
  if (!d->greedy && !d->uniforms) return fail(DSV41_E_INVALID, "sampling requires one uniform per row");
  if (!d->out_ids || !d->out_logprob || !d->out_status)
    return fail(DSV41_E_INVALID, "out_ids, out_logprob and out_status are required");
  const bool pen_on = d->repetition_penalty != 1.0f || d->presence_penalty != 0.0f || d->frequency_penalty != 0.0f;
  const bool hist_given = d->history != nullptr && (d->history_lens != nullptr || d->hist_len > 0);
  if (hist_given) {
    if (d->history_row_stride <= 0) return fail(DSV41_E_INVALID, "history row stride must be positive");
    if (!d->history_lens && (d->hist_len < 0 || d->hist_len > d->history_row_stride))
      return fail(DSV41_E_INVALID, "hist_len must be within the history row stride");
  }
  pl->has_pen = pen_on && hist_given;
  pl->esize = d->logits_dtype == DSV41_DTYPE_F32 ? 4 : 2;
  pl->vec = ((uintptr_t)d->logits % 16 == 0) && ((d->logits_row_stride * pl->esize) % 16 == 0);
  const int V = d->vocab;
  const bool truncating = d->min_p > 0.0f || (d->top_k > 0 && d->top_k < V) || d->top_p < 1.0f;
  if (!truncating) pl->mode = MODE_FULL;
  else if (d->top_k > 0 && d->top_k < V && d->top_k <= KCAP) pl->mode = MODE_TOPK;
  else pl->mode = MODE_GENERIC;
  pl->words = pl->has_pen ? (V + 31) / 32 : 0;
  pl->ucap = pl->has_pen ? (int)std::min<int64_t>(d->history_row_stride, V) : 0;
  Layout L;
  if (pl->mode == MODE_FULL)
    L = pl->esize == 4 ? make_layout<MODE_FULL, 4>(V, pl->words, pl->ucap)
                       : make_layout<MODE_FULL, 8>(V, pl->words, pl->ucap);
  else if (pl->mode == MODE_TOPK)
    L = make_layout<MODE_TOPK, TOPK_G>(V, pl->words, pl->ucap);
  else
    L = make_layout<MODE_GENERIC, 4>(V, pl->words, pl->ucap);
  pl->lds = L.total;
  if (pl->lds > LDS_LIMIT)
    return fail(DSV41_E_UNSUPPORTED, "history length and vocabulary exceed the on-chip penalty tables");
  pl->workspace = pl->mode == MODE_GENERIC ? (size_t)d->rows * (size_t)V * sizeof(float) : 0;
  return DSV41_OK;
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

extern "C" int dsv41_sampler_run(const dsv41_sampler_desc* d, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  Plan pl;
  int rc = plan(d, &pl);
  if (rc != DSV41_OK) return rc;
  if (pl.workspace && (!workspace || workspace_bytes < pl.workspace))
    return fail(DSV41_E_WORKSPACE, "sampler workspace is missing or too small");
  Params p{};
  p.logits = d->logits;
  p.lstride = d->logits_row_stride;
  p.hist = d->history;
  p.hstride = d->history_row_stride;
  p.hlens = d->history_lens;
  p.uniforms = d->uniforms;
  p.out_ids = d->out_ids;
  p.out_lp = d->out_logprob;
  p.out_kept = d->out_kept;
  p.out_status = d->out_status;
  p.zbuf = static_cast<float*>(workspace);
  p.log_min_p = d->min_p > 0.0f ? std::log((double)d->min_p) : -INFINITY;
  p.T = d->temperature;
  p.rT = 1.0f / d->temperature;
  p.rp = d->repetition_penalty;
  p.pres = d->presence_penalty;
  p.freq = d->frequency_penalty;
  p.top_p = d->top_p;
  p.min_p = d->min_p;
  p.V = d->vocab;
  p.hlen = d->hist_len;
  p.top_k = d->top_k;
  p.greedy = d->greedy ? 1 : 0;
  p.has_pen = pl.has_pen ? 1 : 0;
  // z = x / T by the three-operation scheme needs x / T normal and finite for
  // 2^-100 <= |x| < 2^100, which holds for T in [2^-20, 2^20]; other temperatures
  // take IEEE division for every element.
  p.fast_div = (d->temperature >= 0x1p-20f && d->temperature <= 0x1p20f) ? 1 : 0;
  p.unit_T = d->temperature == 1.0f ? 1 : 0;
  p.ucap = pl.ucap;
  p.words = pl.words;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool bf = pl.esize == 2;
  switch (pl.mode) {
    case MODE_FULL:
      if (bf) return pl.vec ? launch(full_kernel<uint16_t, 8, true>, pl.lds, d->rows, p, s)
                            : launch(full_kernel<uint16_t, 8, false>, pl.lds, d->rows, p, s);
      return pl.vec ? launch(full_kernel<float, 4, true>, pl.lds, d->rows, p, s)
                    : launch(full_kernel<float, 4, false>, pl.lds, d->rows, p, s);
    case MODE_TOPK:
      if (bf) return pl.vec ? launch(topk_kernel<uint16_t, true>, pl.lds, d->rows, p, s)
                            : launch(topk_kernel<uint16_t, false>, pl.lds, d->rows, p, s);
      return pl.vec ? launch(topk_kernel<float, true>, pl.lds, d->rows, p, s)
                    : launch(topk_kernel<float, false>, pl.lds, d->rows, p, s);
    default:
      if (bf) return pl.vec ? launch(generic_kernel<uint16_t, 4, true>, pl.lds, d->rows, p, s)
                            : launch(generic_kernel<uint16_t, 4, false>, pl.lds, d->rows, p, s);
      return pl.vec ? launch(generic_kernel<float, 4, true>, pl.lds, d->rows, p, s)
                    : launch(generic_kernel<float, 4, false>, pl.lds, d->rows, p, s);
  }
}
