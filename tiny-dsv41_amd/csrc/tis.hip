// tis.hip — decoupled Token-TIS loss and GRPO loss, their gradients and their diagnostics
// for a packed batch of responses, on gfx950.
//
// Replaces decoupled_token_tis_loss (dsv41_train/rl/algorithm.py:249-346), which loops over
// responses in Python with a few dozen small tensor ops and a host sync per metric, and the
// pooling of its per-response rows (aggregate_token_tis_metrics,
// dsv41_train/rl/distributed_grpo.py:197-222).  Per token i of response r (A = advantage):
//   delta = f32(old - behavior),  raw = exp(f64(delta)),  w = f32(min(raw, cap))
//   ratio = exp(f32(current - old)),  s = min(ratio * A, clamp(ratio, 1 - eps, 1 + eps) * A)
//   loss = mean_r( -mean_{i in r}(w * s) )
// and d loss / d current_i by torch's rules for minimum (ties split the gradient in half)
// and clamp (gradient inside the closed interval).  Metric sums are fp64 over the clamped
// raw weights, as the reference keeps them.
//
// Kernel 1 gives each response one workgroup: a grid-stride pass over its tokens, then a
// fixed-order reduction (wave shuffles, then waves in order), so results repeat bit for bit.
// Kernel 2 folds the per-response partials in a fixed order and writes the loss and the
// metric vector.

#include <math.h>

#include "common.h"

namespace dsv41 {
namespace tis {

constexpr int NT = 256;
constexpr int NW = NT / 64;

struct Part {
  double wsum, wsq, rawsum, dsum, rsum;
  double wmin, wmax, rawmin, rawmax, dmaxabs;
  float term;
  int clipped, rclipped, n;
};

struct Params {
  const int64_t* off;
  const float* cur;
  const float* old;
  const float* beh;
  const float* adv;
  double eps, cap;  // the caller's Python floats
  float lo, hi;     // clamp bounds as torch casts them to the tensor dtype: f32(1 -+ eps)
  int R;
  int64_t T;  // tokens
  Part* part;
  float* grad;
  int32_t* status;
  float* loss;
  double* metrics;
};

template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = op(v, __shfl_xor(v, o));
  return v;
}

// Workgroup reduction in a fixed order: each wave by shuffles, then waves 0..NW-1 in turn.
template <class T, class Op>
__device__ __forceinline__ T block_reduce(T v, Op op, T* scratch) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  v = wave_reduce(v, op);
  if (lane == 0) scratch[wid] = v;
  __syncthreads();
  T r = scratch[0];
  for (int i = 1; i < NW; ++i) r = op(r, scratch[i]);
  __syncthreads();
  return r;
}

struct Add {
  template <class T>
  __device__ T operator()(T a, T b) const { return a + b; }
};
struct Min {
  __device__ double operator()(double a, double b) const { return fmin(a, b); }
};
struct Max {
  __device__ double operator()(double a, double b) const { return fmax(a, b); }
};
struct Or {
  __device__ int operator()(int a, int b) const { return a | b; }
};

__global__ __launch_bounds__(NT) void response_kernel(Params p) {
  __shared__ double sd[NW];
  __shared__ float sf[NW];
  __shared__ int si[NW];
  const int r = blockIdx.x, tid = threadIdx.x;
  const int64_t b0 = p.off[r], e0 = p.off[r + 1];
  int st = 0;
  if (b0 < 0 || e0 > p.T || e0 < b0) st |= DSV41_TIS_BAD_OFFSETS;
  // ranges are clamped to [0, tokens] so that bad offsets cannot read out of bounds
  const int64_t b = min(max(b0, (int64_t)0), p.T), e = min(max(e0, b), p.T);
  const int64_t L = e - b;
  const float A = p.adv[r];
  if (L <= 0) st |= DSV41_TIS_EMPTY;
  if (!isfinite(A)) st |= DSV41_TIS_ADV_NONFINITE;
  const float invL = L > 0 ? 1.0f / (float)L : 0.0f, invR = 1.0f / (float)p.R;
  const float lo = p.lo, hi = p.hi;
  double wsum = 0.0, wsq = 0.0, rawsum = 0.0, dsum = 0.0, rsum = 0.0;
  double wmin = INFINITY, wmax = -INFINITY, rawmin = INFINITY, rawmax = -INFINITY, dmaxabs = 0.0;
  float term = 0.0f;
  int clipped = 0, rclipped = 0;
  for (int64_t i = b + tid; i < e; i += NT) {
    const float c = p.cur[i], o = p.old[i], h = p.beh[i];
    if (!isfinite(c)) st |= DSV41_TIS_CURRENT_NONFINITE;
    else if (c > 1e-6f) st |= DSV41_TIS_CURRENT_POSITIVE;
    if (!isfinite(o)) st |= DSV41_TIS_OLD_NONFINITE;
    else if (o > 1e-6f) st |= DSV41_TIS_OLD_POSITIVE;
    if (!isfinite(h)) st |= DSV41_TIS_BEHAVIOR_NONFINITE;
    else if (h > 1e-6f) st |= DSV41_TIS_BEHAVIOR_POSITIVE;
    const float delta = o - h;
    const double raw = exp((double)delta);
    if (!isfinite(raw)) st |= DSV41_TIS_RAW_NONFINITE;
    else if (raw == 0.0) st |= DSV41_TIS_RAW_ZERO;
    const double wd = fmin(raw, p.cap);
    const float w = (float)wd;
    if (!isfinite(w)) st |= DSV41_TIS_WEIGHT_NONFINITE;
    else if (w == 0.0f) st |= DSV41_TIS_WEIGHT_ZERO;
    const float ratio = expf(c - o);
    if (!isfinite(ratio)) st |= DSV41_TIS_RATIO_NONFINITE;
    else if (ratio == 0.0f) st |= DSV41_TIS_RATIO_ZERO;
    const float u = ratio * A;
    const float rc = fminf(fmaxf(ratio, lo), hi);
    const float cl = rc * A;
    const float s = fminf(u, cl);
    term += w * s;
    if (p.grad) {
      // minimum: the smaller side takes the gradient, ties split it; clamp passes it on [lo, hi]
      const float gu = u < cl ? 1.0f : (u == cl ? 0.5f : 0.0f);
      const float gc = cl < u ? 1.0f : (u == cl ? 0.5f : 0.0f);
      const float inside = (ratio >= lo && ratio <= hi) ? 1.0f : 0.0f;
      const float ds = A * (gu + gc * inside) * ratio;  // d s / d current
      p.grad[i] = -(w * ds) * invL * invR;
    }
    wsum += wd;
    wsq += wd * wd;
    rawsum += raw;
    dsum += (double)delta;
    rsum += (double)ratio;
    wmin = fmin(wmin, wd);
    wmax = fmax(wmax, wd);
    rawmin = fmin(rawmin, raw);
    rawmax = fmax(rawmax, raw);
    dmaxabs = fmax(dmaxabs, fabs((double)delta));
    clipped += raw > p.cap ? 1 : 0;
    rclipped += fabs((double)ratio - 1.0) > p.eps ? 1 : 0;
  }
  wsum = block_reduce(wsum, Add(), sd);
  wsq = block_reduce(wsq, Add(), sd);
  rawsum = block_reduce(rawsum, Add(), sd);
  dsum = block_reduce(dsum, Add(), sd);
  rsum = block_reduce(rsum, Add(), sd);
  wmin = block_reduce(wmin, Min(), sd);
  wmax = block_reduce(wmax, Max(), sd);
  rawmin = block_reduce(rawmin, Min(), sd);
  rawmax = block_reduce(rawmax, Max(), sd);
  dmaxabs = block_reduce(dmaxabs, Max(), sd);
  term = block_reduce(term, Add(), sf);
  clipped = block_reduce(clipped, Add(), si);
  rclipped = block_reduce(rclipped, Add(), si);
  st = block_reduce(st, Or(), si);
  if (tid == 0) {
    Part q;
    q.wsum = wsum;
    q.wsq = wsq;
    q.rawsum = rawsum;
    q.dsum = dsum;
    q.rsum = rsum;
    q.wmin = wmin;
    q.wmax = wmax;
    q.rawmin = rawmin;
    q.rawmax = rawmax;
    q.dmaxabs = dmaxabs;
    q.term = -(term * invL);
    q.clipped = clipped;
    q.rclipped = rclipped;
    q.n = (int)L;
    p.part[r] = q;
    p.status[r] = st;
  }
}

// One workgroup folds the R partials (thread-strided, then block_reduce: a fixed order).
__global__ __launch_bounds__(NT) void pool_kernel(Params p) {
  __shared__ double sd[NW];
  __shared__ float sf[NW];
  __shared__ long long sl[NW];
  const int tid = threadIdx.x;
  double wsum = 0.0, wsq = 0.0, rawsum = 0.0, dsum = 0.0, rsum = 0.0;
  double wmin = INFINITY, wmax = -INFINITY, rawmin = INFINITY, rawmax = -INFINITY, dmaxabs = 0.0;
  float terms = 0.0f;
  long long clipped = 0, rclipped = 0, n = 0;
  for (int r = tid; r < p.R; r += NT) {
    const Part q = p.part[r];
    wsum += q.wsum;
    wsq += q.wsq;
    rawsum += q.rawsum;
    dsum += q.dsum;
    rsum += q.rsum;
    wmin = fmin(wmin, q.wmin);
    wmax = fmax(wmax, q.wmax);
    rawmin = fmin(rawmin, q.rawmin);
    rawmax = fmax(rawmax, q.rawmax);
    dmaxabs = fmax(dmaxabs, q.dmaxabs);
    terms += q.term;
    clipped += q.clipped;
    rclipped += q.rclipped;
    n += q.n;
  }
  wsum = block_reduce(wsum, Add(), sd);
  wsq = block_reduce(wsq, Add(), sd);
  rawsum = block_reduce(rawsum, Add(), sd);
  dsum = block_reduce(dsum, Add(), sd);
  rsum = block_reduce(rsum, Add(), sd);
  wmin = block_reduce(wmin, Min(), sd);
  wmax = block_reduce(wmax, Max(), sd);
  rawmin = block_reduce(rawmin, Min(), sd);
  rawmax = block_reduce(rawmax, Max(), sd);
  dmaxabs = block_reduce(dmaxabs, Max(), sd);
  terms = block_reduce(terms, Add(), sf);
  clipped = block_reduce(clipped, Add(), sl);
  rclipped = block_reduce(rclipped, Add(), sl);
  n = block_reduce(n, Add(), sl);
  if (tid != 0) return;
  const float loss = terms / (float)p.R;
  if (p.loss) p.loss[0] = loss;
  if (!p.metrics) return;
  const double tokens = (double)n, dropped = fmax(rawsum - wsum, 0.0), ess = wsum * wsum / wsq;
  double* m = p.metrics;
  m[DSV41_TIS_M_LOSS] = (double)loss;
  m[DSV41_TIS_M_POLICY_LOSS] = (double)loss;
  m[DSV41_TIS_M_RESPONSE_COUNT] = (double)p.R;
  m[DSV41_TIS_M_TOKEN_COUNT] = tokens;
  m[DSV41_TIS_M_IS_CAP] = p.cap;
  m[DSV41_TIS_M_WEIGHT_SUM] = wsum;
  m[DSV41_TIS_M_WEIGHT_SQUARE_SUM] = wsq;
  m[DSV41_TIS_M_WEIGHT_MEAN] = wsum / tokens;
  m[DSV41_TIS_M_WEIGHT_MIN] = wmin;
  m[DSV41_TIS_M_WEIGHT_MAX] = wmax;
  m[DSV41_TIS_M_RAW_WEIGHT_SUM] = rawsum;
  m[DSV41_TIS_M_RAW_WEIGHT_MIN] = rawmin;
  m[DSV41_TIS_M_RAW_WEIGHT_MAX] = rawmax;
  m[DSV41_TIS_M_CLIPPED_TOKENS] = (double)clipped;
  m[DSV41_TIS_M_CLIPPED_FRACTION] = (double)clipped / tokens;
  m[DSV41_TIS_M_DROPPED_MASS] = dropped;
  m[DSV41_TIS_M_DROPPED_MASS_FRACTION] = dropped / rawsum;
  m[DSV41_TIS_M_ESS] = ess;
  m[DSV41_TIS_M_ESS_FRACTION] = ess / tokens;
  m[DSV41_TIS_M_DELTA_MEAN] = dsum / tokens;
  m[DSV41_TIS_M_DELTA_MAX_ABS] = dmaxabs;
  m[DSV41_TIS_M_RATIO_MEAN] = rsum / tokens;
  m[DSV41_TIS_M_RATIO_CLIP_FRACTION] = (double)rclipped / tokens;
}

// ---------------------------------------------------------------------------- GRPO
// grpo_loss (dsv41_train/rl/algorithm.py:169-246): per response r with A = advantage,
//   ratio = exp(f32(current - behavior)),  s = min(ratio A, clamp(ratio, 1 - eps, 1 + eps) A)
//   k3 = ratio * (expm1(ref - current) - (ref - current))                 (when kl_beta > 0)
//   loss = mean_r(-mean_i s) + kl_beta * mean_r(mean_i k3)
// with d k3 / d current = ratio * (current - ref); metrics are means over responses of the
// per-response means (clip fraction, ratio, -log ratio), all fp32 like the reference's.
struct GPart {
  float pol, kl, clipf, ratio, akl;
};

struct GParams {
  const int64_t* off;
  const float* cur;
  const float* beh;
  const float* ref;
  const float* adv;
  double eps;
  float lo, hi, epsf, beta;
  int R;
  int64_t T;
  GPart* part;
  float* grad;
  int32_t* status;
  float* loss;
  double* metrics;
};

__global__ __launch_bounds__(NT) void grpo_response_kernel(GParams p) {
  __shared__ float sf[NW];
  __shared__ int si[NW];
  const int r = blockIdx.x, tid = threadIdx.x;
  const int64_t b0 = p.off[r], e0 = p.off[r + 1];
  int st = 0;
  if (b0 < 0 || e0 > p.T || e0 < b0) st |= DSV41_GRPO_BAD_OFFSETS;
  const int64_t b = min(max(b0, (int64_t)0), p.T), e = min(max(e0, b), p.T);
  const int64_t L = e - b;
  const float A = p.adv[r];
  if (L <= 0) st |= DSV41_GRPO_EMPTY;
  if (!isfinite(A)) st |= DSV41_GRPO_ADV_NONFINITE;
  const float invL = L > 0 ? 1.0f / (float)L : 0.0f, invR = 1.0f / (float)p.R;
  float pol = 0.0f, kl = 0.0f, clip = 0.0f, rs = 0.0f, akl = 0.0f;
  for (int64_t i = b + tid; i < e; i += NT) {
    const float c = p.cur[i], h = p.beh[i];
    if (!isfinite(c)) st |= DSV41_GRPO_CURRENT_NONFINITE;
    if (!isfinite(h)) st |= DSV41_GRPO_BEHAVIOR_NONFINITE;
    const float lr = c - h;
    const float ratio = expf(lr);
    if (!isfinite(ratio)) st |= DSV41_GRPO_RATIO_NONFINITE;
    const float u = ratio * A;
    const float cl = fminf(fmaxf(ratio, p.lo), p.hi) * A;
    pol += fminf(u, cl);
    clip += fabsf(ratio - 1.0f) > p.epsf ? 1.0f : 0.0f;
    rs += ratio;
    akl += -lr;
    float g = 0.0f;
    if (p.grad) {
      const float gu = u < cl ? 1.0f : (u == cl ? 0.5f : 0.0f);
      const float gc = cl < u ? 1.0f : (u == cl ? 0.5f : 0.0f);
      const float inside = (ratio >= p.lo && ratio <= p.hi) ? 1.0f : 0.0f;
      g = -(A * (gu + gc * inside) * ratio);  // d(-s)/d current
    }
    if (p.ref) {
      const float rf = p.ref[i];
      if (!isfinite(rf)) st |= DSV41_GRPO_REFERENCE_NONFINITE;
      const float delta = rf - c;
      const float k3 = ratio * (expm1f(delta) - delta);
      if (!isfinite(k3)) st |= DSV41_GRPO_K3_NONFINITE;
      kl += k3;
      g += p.beta * (ratio * (c - rf));
    }
    if (p.grad) p.grad[i] = g * invL * invR;
  }
  pol = block_reduce(pol, Add(), sf);
  kl = block_reduce(kl, Add(), sf);
  clip = block_reduce(clip, Add(), sf);
  rs = block_reduce(rs, Add(), sf);
  akl = block_reduce(akl, Add(), sf);
  st = block_reduce(st, Or(), si);
  if (tid == 0) {
    GPart q;
    q.pol = -(pol * invL);
    q.kl = kl * invL;
    q.clipf = clip * invL;
    q.ratio = rs * invL;
    q.akl = akl * invL;
    p.part[r] = q;
    p.status[r] = st;
  }
}

__global__ __launch_bounds__(NT) void grpo_pool_kernel(GParams p) {
  __shared__ float sf[NW];
  const int tid = threadIdx.x;
  float pol = 0.0f, kl = 0.0f, clip = 0.0f, rs = 0.0f, akl = 0.0f;
  for (int r = tid; r < p.R; r += NT) {
    const GPart q = p.part[r];
    pol += q.pol;
    kl += q.kl;
    clip += q.clipf;
    rs += q.ratio;
    akl += q.akl;
  }
  pol = block_reduce(pol, Add(), sf);
  kl = block_reduce(kl, Add(), sf);
  clip = block_reduce(clip, Add(), sf);
  rs = block_reduce(rs, Add(), sf);
  akl = block_reduce(akl, Add(), sf);
  if (tid != 0) return;
  const float invR = 1.0f / (float)p.R;
  const float policy = pol * invR, klm = kl * invR;
  const float loss = policy + p.beta * klm;
  if (p.loss) p.loss[0] = loss;
  if (!p.metrics) return;
  double* m = p.metrics;
  m[DSV41_GRPO_M_LOSS] = (double)loss;
  m[DSV41_GRPO_M_POLICY_LOSS] = (double)policy;
  m[DSV41_GRPO_M_KL] = (double)klm;
  m[DSV41_GRPO_M_CLIP_FRACTION] = (double)(clip * invR);
  m[DSV41_GRPO_M_IMPORTANCE_RATIO] = (double)(rs * invR);
  m[DSV41_GRPO_M_APPROX_KL] = (double)(akl * invR);
}

int plan_grpo(const dsv41_grpo_desc* d, size_t* ws) {
  if (!d) return fail(DSV41_E_INVALID, "GRPO descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_grpo_desc))
    return fail(DSV41_E_ABI, "dsv41_grpo_desc size mismatch (rebuild the binding)");
  if (d->n_responses <= 0 || d->n_tokens < 0)
    return fail(DSV41_E_INVALID, "policy and behavior must contain the same nonzero number of responses");
  if (!(isfinite(d->clip_eps) && d->clip_eps >= 0.0 && d->clip_eps < 1.0))
    return fail(DSV41_E_INVALID, "clip_eps must be finite and in [0, 1)");
  if (!(isfinite(d->kl_beta) && d->kl_beta >= 0.0)) return fail(DSV41_E_INVALID, "kl_beta must be finite and nonnegative");
  if (d->kl_beta > 0.0 && !d->reference)
    return fail(DSV41_E_INVALID, "positive kl_beta requires reference log probabilities");
  if (!d->offsets || !d->current || !d->behavior || !d->advantages || !d->out_status)
    return fail(DSV41_E_INVALID, "offsets, current, behavior, advantages and out_status are required");
  *ws = (size_t)d->n_responses * sizeof(GPart);
  return DSV41_OK;
}

int plan(const dsv41_token_tis_desc* d, size_t* ws) {
  if (!d) return fail(DSV41_E_INVALID, "Token-TIS descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_token_tis_desc))
    return fail(DSV41_E_ABI, "dsv41_token_tis_desc size mismatch (rebuild the binding)");
  if (d->n_responses <= 0 || d->n_tokens < 0)
    return fail(DSV41_E_INVALID, "current, native-old and behavior require the same nonzero response count");
  if (!(isfinite(d->clip_eps) && d->clip_eps >= 0.0 && d->clip_eps < 1.0))
    return fail(DSV41_E_INVALID, "clip_eps must be finite and in [0, 1)");
  if (!(isfinite(d->is_cap) && d->is_cap > 0.0)) return fail(DSV41_E_INVALID, "is_cap must be finite and positive");
  if (!d->offsets || !d->current || !d->native_old || !d->behavior || !d->advantages || !d->out_status)
    return fail(DSV41_E_INVALID, "offsets, the three log-probability vectors, advantages and out_status are required");
  *ws = (size_t)d->n_responses * sizeof(Part);
  return DSV41_OK;
}

}  // namespace tis
}  // namespace dsv41

using namespace dsv41;

extern "C" size_t dsv41_token_tis_workspace_bytes(const dsv41_token_tis_desc* d) {
  size_t ws = 0;
  if (tis::plan(d, &ws) != DSV41_OK) return 0;
  return ws;
}

extern "C" int dsv41_token_tis_run(const dsv41_token_tis_desc* d, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  size_t need = 0;
  int rc = tis::plan(d, &need);
  if (rc != DSV41_OK) return rc;
  if (!workspace || workspace_bytes < need) return fail(DSV41_E_WORKSPACE, "Token-TIS workspace is missing or too small");
  tis::Params p{};
  p.off = d->offsets;
  p.cur = d->current;
  p.old = d->native_old;
  p.beh = d->behavior;
  p.adv = d->advantages;
  p.eps = d->clip_eps;
  p.cap = d->is_cap;
  p.lo = (float)(1.0 - d->clip_eps);
  p.hi = (float)(1.0 + d->clip_eps);
  p.R = d->n_responses;
  p.T = d->n_tokens;
  p.part = static_cast<tis::Part*>(workspace);
  p.grad = d->out_grad;
  p.status = d->out_status;
  p.loss = d->out_loss;
  p.metrics = d->out_metrics;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(tis::response_kernel, dim3(p.R), dim3(tis::NT), 0, s, p);
  DSV41_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(tis::pool_kernel, dim3(1), dim3(tis::NT), 0, s, p);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}

extern "C" size_t dsv41_grpo_workspace_bytes(const dsv41_grpo_desc* d) {
  size_t ws = 0;
  if (tis::plan_grpo(d, &ws) != DSV41_OK) return 0;
  return ws;
}

extern "C" int dsv41_grpo_run(const dsv41_grpo_desc* d, void* workspace, size_t workspace_bytes, void* stream) {
  size_t need = 0;
  int rc = tis::plan_grpo(d, &need);
  if (rc != DSV41_OK) return rc;
  if (!workspace || workspace_bytes < need) return fail(DSV41_E_WORKSPACE, "GRPO workspace is missing or too small");
  tis::GParams p{};
  p.off = d->offsets;
  p.cur = d->current;
  p.beh = d->behavior;
  p.ref = d->kl_beta > 0.0 ? d->reference : nullptr;
  p.adv = d->advantages;
  p.eps = d->clip_eps;
  p.lo = (float)(1.0 - d->clip_eps);
  p.hi = (float)(1.0 + d->clip_eps);
  p.epsf = (float)d->clip_eps;
  p.beta = (float)d->kl_beta;
  p.R = d->n_responses;
  p.T = d->n_tokens;
  p.part = static_cast<tis::GPart*>(workspace);
  p.grad = d->out_grad;
  p.status = d->out_status;
  p.loss = d->out_loss;
  p.metrics = d->out_metrics;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(tis::grpo_response_kernel, dim3(p.R), dim3(tis::NT), 0, s, p);
  DSV41_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(tis::grpo_pool_kernel, dim3(1), dim3(tis::NT), 0, s, p);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}
