// logprob.hip — fused selected-token log-prob for gfx950 (bf16 MFMA).
//
// Replaces DeepSeekV41ForCausalLM._token_log_probs (dsv41_train/models/dsv4/model.py:679-684)
// and ResponseScoringModel._score_targets (dsv41_train/rl/native_lora.py:80-82):
//   logits = x @ w.T (fp32 accumulation, never written out), z = logits / T,
//   logprob[n] = z[n, t_n] - LSE(z[n, :]),  entropy[n] = LSE - sum softmax(z) * z,
// plus the Token-TIS weight of dsv41_train/rl/algorithm.py:293-299 when behaviour
// log-probs are given.
//
// The contraction is computed transposed, C^T[v, n] = sum_k w[v, k] x[n, k], so that an
// MFMA lane owns one token column and the per-token softmax state lives in registers:
// each lane of a 32x32 output block holds 16 vocabulary rows of one token.  A workgroup
// owns BT tokens and sweeps a slice of the vocabulary in BV-row blocks; after each
// block its fp32 accumulators update a running (max, sum e, sum e*z, z_target) per
// token, and slices are merged by a second kernel.
//
// Operands move from HBM to LDS with buffer loads that write LDS directly (no register
// staging), into two stage buffers so the next stage loads while this one multiplies.
// Each 128-byte LDS row holds 64 bf16 of one matrix row with its 16-byte chunks
// XOR-swizzled by (row & 7), so the MFMA fragment reads of 8 consecutive rows hit 8
// different bank groups.

#include <math.h>

#include "common.h"

namespace dsv41 {
namespace logprob {

constexpr int NT = 256;     // 4 waves, 2 (vocab) x 2 (tokens)
constexpr int WV = 4;       // 32-row MFMA blocks per wave along the vocabulary
constexpr int WT = 2;       // 32-column MFMA blocks per wave along tokens
constexpr int BV = 2 * WV * 32;  // 256 vocabulary rows per block
constexpr int BT = 2 * WT * 32;  // tokens per workgroup
constexpr int BK = 64;      // hidden elements per stage (128 bytes per row)
constexpr int STAGE_BYTES = (BV + BT) * 128;
constexpr int LDS_BYTES = 2 * STAGE_BYTES;  // two stage buffers
constexpr float LOG2E = 1.4426950408889634f;
constexpr float NEG_INF = -__builtin_huge_valf();

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

struct Params {
  const uint16_t* x;
  int64_t xs;
  const uint16_t* w;
  int64_t ws;
  const int64_t* targets;
  float4* part;  // [splits][N] (max, sum e, sum e*z, z_target or NaN)
  int N, H, V;
  float invT;
  int splits, vb_per_split, n_vb, n_tb;
  int group_t, group_s;  // XCD super-tile shape (0: linear mapping)
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// merge two softmax states (max, sum e, sum e*z)
__device__ __forceinline__ void merge(float& m, float& s, float& a, float m2, float s2, float a2) {
  const float mn = fmaxf(m, m2);
  if (mn == NEG_INF) return;
  const float c1 = exp2f((m - mn) * LOG2E), c2 = exp2f((m2 - mn) * LOG2E);
  s = s * c1 + s2 * c2;
  a = a * c1 + a2 * c2;
  m = mn;
}

// Block id -> (token block, vocabulary split).  Workgroups are dispatched round-robin
// over the 8 XCDs; consecutive workgroups of one XCD form a group_t x group_s
// rectangle of the (token block, split) grid, so they share operand panels in that
// XCD's L2.  Falls back to split-fastest order when the grid does not tile.
__device__ __forceinline__ void block_coords(const Params& p, int b, int& tb, int& split) {
  const int total = p.n_tb * p.splits;
  if (p.group_t > 0 && total % 8 == 0) {
    const int xcd = b & 7, k = b >> 3;
    const int gsz = p.group_t * p.group_s;
    const int u = (k / gsz) * 8 + xcd;      // super tile index
    const int in = k % gsz;
    const int us_n = p.splits / p.group_s;  // super tiles along splits
    tb = (u / us_n) * p.group_t + in / p.group_s;
    split = (u % us_n) * p.group_s + in % p.group_s;
  } else {
    split = b % p.splits;
    tb = b / p.splits;
  }
}

__global__ __launch_bounds__(NT, 1) void fused_kernel(Params p) {
  __shared__ __align__(16) unsigned char lds[LDS_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wv = wid & 1, wt = wid >> 1;
  int tb, split;
  block_coords(p, blockIdx.x, tb, split);
  const int t0 = tb * BT;
  const int vb0 = split * p.vb_per_split;
  const int vb1 = min(vb0 + p.vb_per_split, p.n_vb);

  // token columns of this lane and their targets
  int tgt[WT];
  float m_[WT], s_[WT], a_[WT], zt_[WT];
#pragma unroll
  for (int j = 0; j < WT; ++j) {
    const int n = t0 + wt * (WT * 32) + j * 32 + (lane & 31);
    tgt[j] = n < p.N ? (int)p.targets[n] : -1;
    m_[j] = NEG_INF;
    s_[j] = 0.0f;
    a_[j] = 0.0f;
    zt_[j] = __builtin_nanf("");
  }

  const int rows_x = min(BT, p.N - t0);
  const __amdgpu_buffer_rsrc_t rx = rsrc(p.x + (int64_t)t0 * p.xs, (uint32_t)(rows_x * p.xs * 2));
  const int nst = (p.H + BK - 1) / BK;

  // Wave w loads rows [w*BV/4, (w+1)*BV/4) of the weight block and rows
  // [w*BT/4, (w+1)*BT/4) of the token block, 8 rows of 128 bytes per instruction.
  // Lane l fills slot l%8 of row l/8, which holds global chunk (l%8) ^ (row & 7).
  constexpr int A_ROWS = BV / 4, B_ROWS = BT / 4;
  static_assert(A_ROWS % 8 == 0 && B_ROWS % 8 == 0, "whole instructions per wave");
  const int lrow = lane >> 3, lslot = lane & 7;
  auto issue_stage = [&](__amdgpu_buffer_rsrc_t rw, int st, int buf) {
    const int k0 = st * BK;
    unsigned char* base = lds + buf * STAGE_BYTES;
#pragma unroll
    for (int q = 0; q < A_ROWS / 8; ++q) {
      const int row = wid * A_ROWS + q * 8 + lrow;
      const int kc = k0 + ((lslot ^ (row & 7)) << 3);
      // chunks past the hidden size get bit 31 set: beyond every row, so they read zero
      const uint32_t off = (uint32_t)((row * p.ws + kc) * 2) | ((uint32_t)(kc >= p.H) << 31);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)(base + (wid * A_ROWS + q * 8) * 128), 16, off, 0,
                                               0, 0);
    }
#pragma unroll
    for (int q = 0; q < B_ROWS / 8; ++q) {
      const int row = wid * B_ROWS + q * 8 + lrow;
      const int kc = k0 + ((lslot ^ (row & 7)) << 3);
      const uint32_t off = (uint32_t)((row * p.xs + kc) * 2) | ((uint32_t)(kc >= p.H) << 31);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(base + BV * 128 + (wid * B_ROWS + q * 8) * 128), 16,
                                               off, 0, 0, 0);
    }
  };

  for (int vb = vb0; vb < vb1; ++vb) {
    const int v0 = vb * BV;
    const int rows_w = min(BV, p.V - v0);
    const __amdgpu_buffer_rsrc_t rw = rsrc(p.w + (int64_t)v0 * p.ws, (uint32_t)(rows_w * p.ws * 2));
    floatx16 acc[WV][WT];
#pragma unroll
    for (int i = 0; i < WV; ++i)
#pragma unroll
      for (int j = 0; j < WT; ++j) acc[i][j] = floatx16{};

    __syncthreads();  // the previous block's last stage has been read
    issue_stage(rw, 0, 0);
    for (int st = 0; st < nst; ++st) {
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's stage data is in LDS
      __syncthreads();                     // all waves' data in; buffer st+1 is free
      if (st + 1 < nst) issue_stage(rw, st + 1, (st + 1) & 1);
      const unsigned char* A = lds + (st & 1) * STAGE_BYTES;
      const unsigned char* B = A + BV * 128;
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        const int c = ks * 2 + (lane >> 5);  // chunk of this lane's 8 values
        bf16x8 fa[WV], fb[WT];
#pragma unroll
        for (int i = 0; i < WV; ++i) {
          const int row = wv * (WV * 32) + i * 32 + (lane & 31);
          fa[i] = *reinterpret_cast<const bf16x8*>(A + row * 128 + ((c ^ (row & 7)) << 4));
        }
#pragma unroll
        for (int j = 0; j < WT; ++j) {
          const int row = wt * (WT * 32) + j * 32 + (lane & 31);
          fb[j] = *reinterpret_cast<const bf16x8*>(B + row * 128 + ((c ^ (row & 7)) << 4));
        }
#pragma unroll
        for (int i = 0; i < WV; ++i)
#pragma unroll
          for (int j = 0; j < WT; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
    }

    // epilogue: lane holds rows 8*(r/4) + 4*(lane/32) + r%4 of each 32-row block; the
    // running state absorbs one 16-value block at a time
    // positions are compared relative to this lane's first row, so each (i, r) is a
    // compile-time offset
    const int rbase = v0 + wv * (WV * 32) + 4 * (lane >> 5);
    const int lim = p.V - rbase;  // offsets below lim are rows of the vocabulary
#pragma unroll
    for (int j = 0; j < WT; ++j) {
      const int dt = tgt[j] - rbase;
#pragma unroll
      for (int i = 0; i < WV; ++i) {
        float z[16];
        float mx = NEG_INF;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int off = i * 32 + 8 * (r >> 2) + (r & 3);
          z[r] = off < lim ? acc[i][j][r] * p.invT : NEG_INF;
          mx = fmaxf(mx, z[r]);
          if (off == dt) zt_[j] = z[r];
        }
        const float mn = fmaxf(m_[j], mx);
        if (mn == NEG_INF) continue;
        const float cs = exp2f((m_[j] - mn) * LOG2E);
        const float mb = mn * LOG2E;
        float s = 0.0f, a = 0.0f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = exp2f(__builtin_fmaf(z[r], LOG2E, -mb));
          s += e;
          a = __builtin_fmaf(e, z[r] == NEG_INF ? 0.0f : z[r], a);
        }
        s_[j] = __builtin_fmaf(s_[j], cs, s);
        a_[j] = __builtin_fmaf(a_[j], cs, a);
        m_[j] = mn;
      }
    }
  }

  // combine the two lane halves (same tokens, interleaved rows), then the two vocab waves
#pragma unroll
  for (int j = 0; j < WT; ++j) {
    const float m2 = __shfl_xor(m_[j], 32), s2 = __shfl_xor(s_[j], 32), a2 = __shfl_xor(a_[j], 32);
    const float z2 = __shfl_xor(zt_[j], 32);
    merge(m_[j], s_[j], a_[j], m2, s2, a2);
    if (zt_[j] != zt_[j]) zt_[j] = z2;
  }
  __syncthreads();
  float4* xch = reinterpret_cast<float4*>(lds);  // [2 (wt)][WT*32] states of wave wv = 1
  if (wv == 1 && lane < 32) {
#pragma unroll
    for (int j = 0; j < WT; ++j) xch[wt * (WT * 32) + j * 32 + lane] = make_float4(m_[j], s_[j], a_[j], zt_[j]);
  }
  __syncthreads();
  if (wv == 0 && lane < 32) {
#pragma unroll
    for (int j = 0; j < WT; ++j) {
      const float4 o = xch[wt * (WT * 32) + j * 32 + lane];
      merge(m_[j], s_[j], a_[j], o.x, o.y, o.z);
      if (zt_[j] != zt_[j]) zt_[j] = o.w;
      const int n = t0 + wt * (WT * 32) + j * 32 + lane;
      if (n < p.N) p.part[(int64_t)split * p.N + n] = make_float4(m_[j], s_[j], a_[j], zt_[j]);
    }
  }
}

struct MergeParams {
  const float4* part;
  int N, splits;
  const float* behavior;
  float is_cap;
  float* lp;
  float* ent;
  float* ratio;
  int32_t* status;
};

__global__ __launch_bounds__(256) void merge_kernel(MergeParams q) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= q.N) return;
  float m = NEG_INF, s = 0.0f, a = 0.0f, zt = __builtin_nanf("");
  for (int k = 0; k < q.splits; ++k) {
    const float4 o = q.part[(int64_t)k * q.N + n];
    merge(m, s, a, o.x, o.y, o.z);
    if (zt != zt) zt = o.w;
  }
  const float lse = m + logf(s);
  const float lp = zt - lse;
  const float ent = lse - a / s;
  int st = 0;
  if (!isfinite(lp) || !isfinite(ent)) st |= DSV41_STATUS_NONFINITE;
  q.lp[n] = lp;
  if (q.ent) q.ent[n] = ent;
  if (q.ratio) {
    // algorithm.py:293-299: delta in fp32, exp in fp64, clamp at the cap, back to fp32
    const float delta = lp - q.behavior[n];
    const double raw = exp((double)delta);
    if (raw == 0.0) st |= DSV41_STATUS_RATIO_ZERO;
    if (!isfinite(raw)) st |= DSV41_STATUS_NONFINITE;
    q.ratio[n] = (float)fmin((double)q.is_cap, raw);
  }
  if (q.status) q.status[n] = st;
}

struct Plan {
  int splits, vb_per_split, n_vb, n_tb, group_t, group_s;
  size_t workspace;
};

int plan(const dsv41_logprob_desc* d, Plan* pl) {
  if (!d) return fail(DSV41_E_INVALID, "log-prob descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_logprob_desc))
    return fail(DSV41_E_ABI, "dsv41_logprob_desc size mismatch (rebuild the binding)");
  if (d->n_tokens < 0 || d->hidden <= 0 || d->vocab <= 0)
    return fail(DSV41_E_INVALID, "hidden states must be [tokens, hidden] and the head [vocab, hidden]");
  if (d->hidden % 8 != 0) return fail(DSV41_E_UNSUPPORTED, "hidden size must be a multiple of 8");
  if (d->x_row_stride < d->hidden || d->w_row_stride < d->hidden || d->x_row_stride % 8 || d->w_row_stride % 8)
    return fail(DSV41_E_INVALID, "row strides must be >= hidden and multiples of 8 elements");
  if (((uintptr_t)d->x | (uintptr_t)d->w) % 16)
    return fail(DSV41_E_INVALID, "hidden states and head weight must be 16-byte aligned");
  if ((int64_t)BV * d->w_row_stride * 2 >= (1ll << 31) || (int64_t)BT * d->x_row_stride * 2 >= (1ll << 31))
    return fail(DSV41_E_UNSUPPORTED, "row stride too large for 32-bit block offsets");
  if (!(isfinite(d->temperature) && d->temperature > 0.0f))
    return fail(DSV41_E_INVALID, "temperature must be finite and positive");
  if (d->out_ratio && !d->behavior) return fail(DSV41_E_INVALID, "ratio output requires behavior log-probs");
  if (d->behavior && !(isfinite(d->is_cap) && d->is_cap > 0.0f))
    return fail(DSV41_E_INVALID, "is_cap must be finite and positive");
  if (d->n_tokens > 0 && (!d->x || !d->w || !d->targets || !d->out_logprob))
    return fail(DSV41_E_INVALID, "x, w, targets and out_logprob are required");
  pl->n_vb = (d->vocab + BV - 1) / BV;
  pl->n_tb = (d->n_tokens + BT - 1) / BT;
  // about four workgroups per CU across the machine, at least one vocabulary block each
  const int want = pl->n_tb > 0 ? (1024 + pl->n_tb - 1) / pl->n_tb : 1;
  pl->splits = std::max(1, std::min(want, pl->n_vb));
  pl->vb_per_split = (pl->n_vb + pl->splits - 1) / pl->splits;
  pl->splits = (pl->n_vb + pl->vb_per_split - 1) / pl->vb_per_split;
  // XCD super tiles of 32 workgroups (token blocks x splits) when the grid tiles
  pl->group_t = 0;
  pl->group_s = 0;
  for (int gs : {8, 4, 16, 2, 32}) {
    const int gt = 32 / gs;
    if (pl->splits % gs == 0 && pl->n_tb % gt == 0 && (pl->n_tb * pl->splits) % (8 * 32) == 0) {
      pl->group_t = gt;
      pl->group_s = gs;
      break;
    }
  }
  pl->workspace = (size_t)pl->splits * (size_t)d->n_tokens * sizeof(float4);
  return DSV41_OK;
}

}  // namespace logprob
}  // namespace dsv41

using namespace dsv41;
using namespace dsv41::logprob;

extern "C" size_t dsv41_logprob_workspace_bytes(const dsv41_logprob_desc* d) {
  Plan pl;
  if (plan(d, &pl) != DSV41_OK) return 0;
  return pl.workspace;
}

extern "C" int dsv41_logprob_run(const dsv41_logprob_desc* d, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  Plan pl;
  int rc = plan(d, &pl);
  if (rc != DSV41_OK) return rc;
  if (d->n_tokens == 0) return DSV41_OK;
  if (!workspace || workspace_bytes < pl.workspace)
    return fail(DSV41_E_WORKSPACE, "log-prob workspace is missing or too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Params p{};
  p.x = static_cast<const uint16_t*>(d->x);
  p.xs = d->x_row_stride;
  p.w = static_cast<const uint16_t*>(d->w);
  p.ws = d->w_row_stride;
  p.targets = d->targets;
  p.part = static_cast<float4*>(workspace);
  p.N = d->n_tokens;
  p.H = d->hidden;
  p.V = d->vocab;
  p.invT = 1.0f / d->temperature;
  p.splits = pl.splits;
  p.vb_per_split = pl.vb_per_split;
  p.n_vb = pl.n_vb;
  p.n_tb = pl.n_tb;
  p.group_t = pl.group_t;
  p.group_s = pl.group_s;
  hipLaunchKernelGGL(fused_kernel, dim3(pl.n_tb * pl.splits), dim3(NT), 0, s, p);
  DSV41_HIP_CHECK(hipGetLastError());
  MergeParams q{};
  q.part = p.part;
  q.N = d->n_tokens;
  q.splits = pl.splits;
  q.behavior = d->behavior;
  q.is_cap = d->is_cap;
  q.lp = d->out_logprob;
  q.ent = d->out_entropy;
  q.ratio = d->out_ratio;
  q.status = d->out_status;
  hipLaunchKernelGGL(merge_kernel, dim3((d->n_tokens + 255) / 256), dim3(256), 0, s, q);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}
