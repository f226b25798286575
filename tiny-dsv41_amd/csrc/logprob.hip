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
// owns BT = 256 tokens and sweeps a range of the vocabulary in BV = 256-row blocks (each
// of its eight waves, two per SIMD, computes a 128 x 64 part); after each block the fp32
// accumulators update a running (max, sum e, sum e*z) per token.  A second kernel merges
// the vocabulary ranges and computes the target logit as its own dot product.
//
// Operands move from HBM to LDS with buffer loads that write LDS directly (no register
// staging), into two stage buffers of 64 hidden elements per row: 128 bytes, one whole
// cache line of every row, so each line crosses L2 -> L1 once (with half-line stages
// every line crosses twice, as the L1 cannot keep the other half until the next stage).
// The stage sequence runs straight across vocabulary blocks, so the pipeline never
// drains between blocks.  Each stage has one barrier, after its third k-step: before it
// every wave waits for its own fragment reads of the stage and its own loads of the next
// stage, so after it the next stage is readable by all and the current stage's buffer
// takes the loads of the stage after next, a whole stage ahead of their use.  Those loads
// and the next stage's first fragment reads are slotted between the multiplies of the
// last k-step; the other k-steps carry the fragment reads of the k-step after them.  MFMA
// operand fragments alternate between two register sets, so reads never wait for the
// multiplies that use the other set.  Each 128-byte LDS row holds its eight 16-byte
// chunks XOR-swizzled by (row >> 1) & 7; with that, a wave-wide 16-byte read of one chunk
// of 32 consecutive rows is free of bank conflicts on gfx950's LDS (measured: 4 cycles per
// read, against 8 for row & 7 and 32 unswizzled).

#include <math.h>

#include "common.h"

namespace dsv41 {
namespace logprob {

constexpr int WAVES_V = 2;                   // waves along the vocabulary
constexpr int WAVES_T = 4;                   // waves along tokens
constexpr int NWAVES = WAVES_V * WAVES_T;
constexpr int NT = 64 * NWAVES;              // 8 waves, two per SIMD
constexpr int WV = 4;                        // 32-row MFMA blocks per wave along the vocabulary
constexpr int WT = 2;                        // 32-column MFMA blocks per wave along tokens
constexpr int BV = WAVES_V * WV * 32;        // 256 vocabulary rows per block
constexpr int BT = WAVES_T * WT * 32;        // 256 tokens per workgroup
constexpr int BK = 64;                       // hidden elements per stage
constexpr int KS = BK / 16;                  // MFMA k-steps per stage
constexpr int ROWB = BK * 2;                 // bytes per LDS row: one 128-byte cache line
constexpr int STAGE_BYTES = (BV + BT) * ROWB;  // 64 KiB
constexpr int LDS_BYTES = 2 * STAGE_BYTES;   // two stage buffers
constexpr int ROWS_PER_LOAD = 1024 / ROWB;   // rows one wave-wide 16-byte LDS load fills
constexpr int A_LOADS = BV / NWAVES / ROWS_PER_LOAD;  // per wave per stage
constexpr int B_LOADS = BT / NWAVES / ROWS_PER_LOAD;
constexpr int CU_COUNT = 256;                // MI355X
constexpr float LOG2E = 1.4426950408889634f;
constexpr float NEG_INF = -__builtin_huge_valf();

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

struct Params {
  const uint16_t* x;
  int64_t xs;
  const uint16_t* w;  // (backward: row vbeg of the head)
  int64_t ws;
  const int64_t* targets;
  float4* part;  // [splits][N] (max z, sum e, sum e*z, unused)
  int N, H, V;   // (backward: V = rows of the vocabulary range)
  float invT;
  int splits, n_vb, n_tb;
  int group_t, group_s;  // XCD super-tile shape (0: linear mapping)
  // backward only
  const float* lse;
  const float* ent;
  const float* glp;
  const float* gent;
  uint16_t* out;  // bf16 [N, os]
  int64_t os;
  int vbeg;
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

// Bank-group swizzle of the 16-byte chunks of LDS row `row`.  It depends only on
// row % 16, so every 32-row MFMA block shares one pattern.
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

// s_waitcnt vmcnt(0), expcnt and lgkmcnt left at their maxima: this wave's LDS loads landed.
__device__ __forceinline__ void wait_loads() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier with no memory fence: completion of the LDS loads is tracked with
// wait_loads, and the memory clobber keeps the compiler from moving LDS accesses across.
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void read_frags(const unsigned char* stage, int addr_a, int addr_b, bf16x8 (&fa)[WV],
                                           bf16x8 (&fb)[WT]) {
#pragma unroll
  for (int i = 0; i < WV; ++i) fa[i] = *reinterpret_cast<const bf16x8*>(stage + addr_a + i * 32 * ROWB);
#pragma unroll
  for (int j = 0; j < WT; ++j) fb[j] = *reinterpret_cast<const bf16x8*>(stage + addr_b + j * 32 * ROWB);
}

// One k-step of the wave's WV x WT block of 32x32 outputs, with other work slotted
// between the multiplies: after multiply i,
// extra(i) issues one fragment read or load (each group is fenced so the scheduler
// keeps the interleave).
template <class Extra>
__device__ __forceinline__ void mfma_set_x(floatx16 (&acc)[WV][WT], const bf16x8 (&fa)[WV], const bf16x8 (&fb)[WT],
                                           Extra&& extra) {
#pragma unroll
  for (int i = 0; i < WV; ++i)
#pragma unroll
    for (int j = 0; j < WT; ++j) {
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      extra(i * WT + j);
      __builtin_amdgcn_sched_barrier(0);
    }
}

// Folds one vocabulary block into the running (max z, sum e, sum e*z) of token column j.
// Rows at offsets >= lim lie past the vocabulary (their weights read as zero) and are
// skipped when MASK is set.
template <bool MASK>
__device__ __forceinline__ void absorb(const floatx16 (&acc)[WV][WT], int j, int lim, float invT, float& m,
                                       float& s, float& a) {
  float mx = NEG_INF;
#pragma unroll
  for (int i = 0; i < WV; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int off = i * 32 + 8 * (r >> 2) + (r & 3);
      mx = fmaxf(mx, (!MASK || off < lim) ? acc[i][j][r] : NEG_INF);
    }
  const float mn = fmaxf(m, mx * invT);  // invT > 0: the max commutes with the scaling
  if (mn == NEG_INF) return;
  const float c1 = invT * LOG2E, mb = mn * LOG2E;
  float sum = 0.0f, ea = 0.0f;
#pragma unroll
  for (int i = 0; i < WV; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int off = i * 32 + 8 * (r >> 2) + (r & 3);
      const float v = acc[i][j][r];
      const float e = exp2f((!MASK || off < lim) ? __builtin_fmaf(v, c1, -mb) : NEG_INF);
      sum += e;
      ea = __builtin_fmaf(e, v, ea);
    }
  const float cs = exp2f((m - mn) * LOG2E);
  s = __builtin_fmaf(s, cs, sum);
  a = __builtin_fmaf(a, cs, ea * invT);
  m = mn;
}

// Two floats to bf16 (round to nearest even), packed low | high << 16.
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 v = {(__bf16)lo, (__bf16)hi};
  return __builtin_bit_cast(uint32_t, v);
}

// Backward epilogue of one vocabulary block: dL/dz per element from the recomputed logit,
// scaled by 1/T and rounded to bf16, written straight from the accumulators (each lane
// stores its four consecutive vocabulary rows of a token as 8 bytes; the lines of an
// output row fill up in L2 across the wave's stores).
__device__ __forceinline__ void grad_block(const Params& p, const floatx16 (&acc)[WV][WT], int t0, int vb, int wv,
                                           int wt, int lane) {
  const int r32 = lane & 31, half = lane >> 5;
  const int cols = min(BV, p.V - vb * BV);
#pragma unroll
  for (int j = 0; j < WT; ++j) {
    const int n = t0 + wt * (WT * 32) + j * 32 + r32;
    if (n >= p.N) continue;
    const float lse = p.lse[n];
    const float glp = p.glp ? p.glp[n] : 0.0f;
    const float gent = p.gent ? p.gent[n] : 0.0f;
    const float cent = p.gent ? lse - p.ent[n] : 0.0f;  // lse - entropy = E[z]
    const int64_t tt = p.targets[n] - p.vbeg - (int64_t)vb * BV;
    const int tl = (tt >= 0 && tt < BV) ? (int)tt : -1;  // target row within this block, if there
    const float mb = lse * LOG2E, c1 = p.invT * LOG2E;
    uint16_t* row = p.out + (int64_t)n * p.os + (int64_t)vb * BV;
#pragma unroll
    for (int i = 0; i < WV; ++i)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int v0 = wv * (WV * 32) + i * 32 + 8 * g4 + 4 * half;  // rows v0 .. v0+3
        float gv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = acc[i][j][4 * g4 + e];
          const float z = a * p.invT;
          const float pr = exp2f(__builtin_fmaf(a, c1, -mb));
          const float onehot = (v0 + e == tl) ? 1.0f : 0.0f;
          const float g = glp * (onehot - pr) + gent * pr * (cent - z);
          gv[e] = g * p.invT;
        }
        uint2 w2;
        w2.x = pack_bf16(gv[0], gv[1]);
        w2.y = pack_bf16(gv[2], gv[3]);
        if (v0 + 4 <= cols) {
          *reinterpret_cast<uint2*>(row + v0) = w2;
        } else {  // the vocabulary range ends inside these four rows
          if (v0 < cols) row[v0] = (uint16_t)w2.x;
          if (v0 + 1 < cols) row[v0 + 1] = (uint16_t)(w2.x >> 16);
          if (v0 + 2 < cols) row[v0 + 2] = (uint16_t)w2.y;
        }
      }
  }
}

template <bool GRAD>
__global__ __launch_bounds__(NT, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void fused_kernel(Params p) {
  __shared__ __align__(16) unsigned char lds[LDS_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int wv = wid % WAVES_V, wt = wid / WAVES_V;
  int tb, split;
  block_coords(p, blockIdx.x, tb, split);
  const int t0 = tb * BT;
  const int vb0 = (int)((int64_t)split * p.n_vb / p.splits);
  const int vb1 = (int)((int64_t)(split + 1) * p.n_vb / p.splits);
  const int nst = (p.H + BK - 1) / BK;  // stages per vocabulary block
  const int total = (vb1 - vb0) * nst;  // stages of this workgroup

  float m_[WT], s_[WT], a_[WT];
#pragma unroll
  for (int j = 0; j < WT; ++j) {
    m_[j] = NEG_INF;
    s_[j] = 0.0f;
    a_[j] = 0.0f;
  }

  // Loader.  Wave w fills rows [R*w, R*w + R) of the weight block and of the token block,
  // R = 256 / NWAVES; lane l of load q fills slot l%8 of row R*w + 8q + l/8 with global
  // chunk (l%8) ^ swz(row) = (l%8) ^ swz(l/8) ^ 4*(q%2).  Chunks at or past the hidden
  // size (only in a final partial stage) get bit 31 of the offset set, past every buffer,
  // so they read zero.
  constexpr int R = BV / NWAVES;
  static_assert(BV == BT && R % 16 == 0 && ROWS_PER_LOAD == 8, "loader layout");
  const int rows_x = min(BT, p.N - t0);
  const __amdgpu_buffer_rsrc_t rx = rsrc(p.x + (int64_t)t0 * p.xs, (uint32_t)(rows_x * p.xs * 2));
  const int lrow = wid * R + (lane >> 3);
  const int lch = (lane & 7) ^ swz(lane >> 3);  // global chunk for even q; odd q load lch ^ 4
  const uint32_t la = (uint32_t)(lrow * p.ws * 2), lb = (uint32_t)(lrow * p.xs * 2);
  const uint32_t qa = (uint32_t)(8 * p.ws * 2), qb = (uint32_t)(8 * p.xs * 2);
  int ld = 0, ld_k = 0, ld_vb = vb0;
  auto w_rsrc = [&](int vb) {
    const int v0 = vb * BV;
    return rsrc(p.w + (int64_t)v0 * p.ws, (uint32_t)(min(BV, p.V - v0) * p.ws * 2));
  };
  __amdgpu_buffer_rsrc_t rw_ld = w_rsrc(vb0);
  // The loads of one stage, one instruction per call q = 0 .. A_LOADS + B_LOADS - 1;
  // advance() moves to the next stage afterwards.
  uint32_t c0 = 0, c1 = 0;
  unsigned char* ld_base = lds;
  auto stage_setup = [&]() {
    ld_base = lds + (ld & 1) * STAGE_BYTES;
    const int k0 = ld_k * BK;
    c0 = (uint32_t)((k0 + 8 * lch) * 2);
    c1 = (uint32_t)((k0 + 8 * (lch ^ 4)) * 2);
    if (k0 + BK > p.H) {
      c0 |= (uint32_t)(k0 + 8 * lch >= p.H) << 31;
      c1 |= (uint32_t)(k0 + 8 * (lch ^ 4) >= p.H) << 31;
    }
    if (ld >= total) {  // past the last stage: read nothing
      c0 |= 1u << 31;
      c1 |= 1u << 31;
    }
  };
  auto issue_one = [&](int q) {
    if (q < A_LOADS)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw_ld, (lds_ptr_t)(ld_base + (wid * R + q * 8) * ROWB), 16,
                                               la + q * qa + ((q & 1) ? c1 : c0), 0, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_ptr_t)(ld_base + (BV + wid * R + (q - A_LOADS) * 8) * ROWB),
                                               16, lb + (q - A_LOADS) * qb + (((q - A_LOADS) & 1) ? c1 : c0), 0, 0, 0);
  };
  auto advance = [&]() {
    ++ld;
    if (++ld_k == nst) {
      ld_k = 0;
      if (++ld_vb < vb1) rw_ld = w_rsrc(ld_vb);
    }
  };
  auto issue_next = [&]() {
    stage_setup();
#pragma unroll
    for (int q = 0; q < A_LOADS + B_LOADS; ++q) issue_one(q);
    advance();
  };

  // Fragment reads: lane l takes row l%32 of each 32-row block and 8 values of chunk
  // 2*ks + l/32, stored at slot chunk ^ swz(l%32).
  const int r32 = lane & 31, half = lane >> 5;
  const int fa_base = (wv * (WV * 32) + r32) * ROWB, fb_base = (BV + wt * (WT * 32) + r32) * ROWB;
  int fch[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) fch[ks] = ((2 * ks + half) ^ swz(r32)) << 4;

  // Prologue: stage 0 landed, its first fragments in registers, stage 1 on its way.
  issue_next();
  wait_loads();
  barrier();
  static_assert(KS == 4, "the stage body below is written for four k-steps");
  static_assert(A_LOADS + B_LOADS <= WV * WT && WV + WT <= WV * WT, "interleave slots");
  bf16x8 fa0[WV], fb0[WT], fa1[WV], fb1[WT];
  read_frags(lds, fa_base + fch[0], fb_base + fch[0], fa0, fb0);
  issue_next();

  // One barrier per stage.  Before it every wave has all of its reads of stage st back
  // and its loads of stage st+1 landed, so after it stage st+1 is readable and the
  // buffer of stage st takes the loads of stage st+2, a whole stage ahead of their use.
  // Slot order: both token fragments first, then the weight fragments, so that each read
  // is at least six multiplies ahead of its first use in the next k-step (multiplies run
  // i-major: fb[0], fb[1] and fa[0] are needed first).
  auto frag_read = [&](const unsigned char* stage, int c, bf16x8 (&fa)[WV], bf16x8 (&fb)[WT], int slot) {
    if (slot < WT) fb[slot] = *reinterpret_cast<const bf16x8*>(stage + fb_base + c + slot * 32 * ROWB);
    else if (slot < WV + WT) fa[slot - WT] = *reinterpret_cast<const bf16x8*>(stage + fa_base + c + (slot - WT) * 32 * ROWB);
  };
  int st = 0;  // index of the stage being multiplied in this workgroup's sequence
  for (int vb = vb0; vb < vb1; ++vb) {
    floatx16 acc[WV][WT];
#pragma unroll
    for (int i = 0; i < WV; ++i)
#pragma unroll
      for (int j = 0; j < WT; ++j) acc[i][j] = floatx16{};
    for (int kst = 0; kst < nst; ++kst, ++st) {
      const unsigned char* stage = lds + (st & 1) * STAGE_BYTES;
      mfma_set_x(acc, fa0, fb0, [&](int i) { frag_read(stage, fch[1], fa1, fb1, i); });
      mfma_set_x(acc, fa1, fb1, [&](int i) { frag_read(stage, fch[2], fa0, fb0, i); });
      mfma_set_x(acc, fa0, fb0, [&](int i) { frag_read(stage, fch[3], fa1, fb1, i); });
      __builtin_amdgcn_s_waitcnt(0);  // own reads of stage st back, own loads of stage st+1 landed
      barrier();
      const unsigned char* next = lds + ((st + 1) & 1) * STAGE_BYTES;
      // After the last stage the reads below fetch a buffer nobody uses and the loads
      // read zeros (offsets past the buffer); both stay unconditional so the multiplies
      // see one straight-line sequence.
      stage_setup();
      // Raised priority for the k-step that carries the next loads: the SIMD's two waves
      // leave the barrier together, and the one that falls behind in this k-step wins
      // the issue arbitration until it drops back, so both reach the next barrier
      // together instead of one idling there (measured: 24.5 -> 22.9 ms at D).
      __builtin_amdgcn_s_setprio(1);
      mfma_set_x(acc, fa1, fb1, [&](int i) {
        frag_read(next, fch[0], fa0, fb0, i);
        if (i < A_LOADS + B_LOADS) issue_one(i);
      });
      __builtin_amdgcn_s_setprio(0);
      advance();
    }

    // end of a vocabulary block: lane holds rows 8*(r/4) + 4*(lane/32) + r%4 of each
    // 32-row block, at offsets from rbase that are compile-time constants
    if constexpr (GRAD) {
      grad_block(p, acc, t0, vb, wv, wt, lane);
      continue;
    }
    const int rbase = vb * BV + wv * (WV * 32) + 4 * half;
    if ((vb + 1) * BV <= p.V) {
#pragma unroll
      for (int j = 0; j < WT; ++j) absorb<false>(acc, j, 0, p.invT, m_[j], s_[j], a_[j]);
    } else {
      const int lim = p.V - rbase;
#pragma unroll
      for (int j = 0; j < WT; ++j) absorb<true>(acc, j, lim, p.invT, m_[j], s_[j], a_[j]);
    }
  }

  if constexpr (GRAD) return;
  // combine the two lane halves (same tokens, interleaved rows), then the two vocab waves
#pragma unroll
  for (int j = 0; j < WT; ++j) {
    const float m2 = __shfl_xor(m_[j], 32), s2 = __shfl_xor(s_[j], 32), a2 = __shfl_xor(a_[j], 32);
    merge(m_[j], s_[j], a_[j], m2, s2, a2);
  }
  __builtin_amdgcn_s_waitcnt(0x0F70);  // no LDS loads in flight
  __syncthreads();
  static_assert(WAVES_V == 2, "the exchange below merges two vocabulary waves");
  float4* xch = reinterpret_cast<float4*>(lds);  // [WAVES_T][WT*32] states of the waves with wv = 1
  if (wv == 1 && lane < 32) {
#pragma unroll
    for (int j = 0; j < WT; ++j) xch[wt * (WT * 32) + j * 32 + lane] = make_float4(m_[j], s_[j], a_[j], 0.0f);
  }
  __syncthreads();
  if (wv == 0 && lane < 32) {
#pragma unroll
    for (int j = 0; j < WT; ++j) {
      const float4 o = xch[wt * (WT * 32) + j * 32 + lane];
      merge(m_[j], s_[j], a_[j], o.x, o.y, o.z);
      const int n = t0 + wt * (WT * 32) + j * 32 + lane;
      if (n < p.N) p.part[(int64_t)split * p.N + n] = make_float4(m_[j], s_[j], a_[j], 0.0f);
    }
  }
}

struct MergeParams {
  const float4* part;  // [splits][N] split states, or [shards][N] shard states (combine)
  const uint16_t* x;
  int64_t xs;
  const uint16_t* w;
  int64_t ws;
  const int64_t* targets;
  int N, H, V, splits;
  int64_t voff;  // shard: global id of w's first row
  float invT;
  const float* behavior;
  float is_cap;
  float* lp;
  float* ent;
  float* ratio;
  int32_t* status;
  float* lse_out;
  float4* state_out;  // shard: [N] merged states
};

__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xFFFF0000u); }

constexpr int MERGE_FINAL = 0;    // split states + target dot product -> log-prob, entropy, ratio
constexpr int MERGE_STATE = 1;    // split states + target dot product -> one shard state per token
constexpr int MERGE_COMBINE = 2;  // shard states (target logit inside) -> log-prob, entropy, ratio

// One wave per token.  The target logit z_t = (x[n] . w[t_n]) / T is an fp32 dot product
// (FINAL, and STATE when this shard holds row t_n; -inf otherwise); COMBINE takes it from the
// shard that holds it.  The states merge exactly (associative LSE merge), then log-prob,
// entropy, lse, the Token-TIS weight and status, or (STATE) the merged 16-byte state.
template <int MODE>
__global__ __launch_bounds__(256) void merge_kernel(MergeParams q) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (n >= q.N) return;  // uniform per wave
  float zt = MODE == MERGE_STATE ? NEG_INF : __builtin_nanf("");
  if (MODE != MERGE_COMBINE) {
    const int64_t t = q.targets[n] - q.voff;
    if (t >= 0 && t < q.V) {
      const uint4* xr = reinterpret_cast<const uint4*>(q.x + (int64_t)n * q.xs);
      const uint4* wr = reinterpret_cast<const uint4*>(q.w + t * q.ws);
      float d0 = 0.0f, d1 = 0.0f;
      for (int c = lane; c < q.H / 8; c += 64) {
        const uint4 xv = xr[c], wv = wr[c];
        d0 = __builtin_fmaf(bf16_lo(xv.x), bf16_lo(wv.x), d0);
        d1 = __builtin_fmaf(bf16_hi(xv.x), bf16_hi(wv.x), d1);
        d0 = __builtin_fmaf(bf16_lo(xv.y), bf16_lo(wv.y), d0);
        d1 = __builtin_fmaf(bf16_hi(xv.y), bf16_hi(wv.y), d1);
        d0 = __builtin_fmaf(bf16_lo(xv.z), bf16_lo(wv.z), d0);
        d1 = __builtin_fmaf(bf16_hi(xv.z), bf16_hi(wv.z), d1);
        d0 = __builtin_fmaf(bf16_lo(xv.w), bf16_lo(wv.w), d0);
        d1 = __builtin_fmaf(bf16_hi(xv.w), bf16_hi(wv.w), d1);
      }
      zt = wave_sum(d0 + d1) * q.invT;
    }
  }
  float m = NEG_INF, s = 0.0f, a = 0.0f, zs = NEG_INF;
  for (int k = lane; k < q.splits; k += 64) {
    const float4 o = q.part[(int64_t)k * q.N + n];
    merge(m, s, a, o.x, o.y, o.z);
    if (MODE == MERGE_COMBINE) zs = fmaxf(zs, o.w);
  }
  const float mx = wave_max(m);
  const float c = m == NEG_INF ? 0.0f : exp2f((m - mx) * LOG2E);
  s = wave_sum(s * c);
  a = wave_sum(a * c);
  if (MODE == MERGE_COMBINE) {
    zs = wave_max(zs);
    zt = zs > NEG_INF ? zs : __builtin_nanf("");  // no shard held the target
  }
  if (lane != 0) return;
  if (MODE == MERGE_STATE) {
    q.state_out[n] = make_float4(mx, s, a, zt);
    return;
  }
  const float lse = mx + logf(s);
  const float lp = zt - lse;
  const float ent = lse - a / s;
  int st = 0;
  if (!isfinite(lp) || !isfinite(ent)) st |= DSV41_STATUS_NONFINITE;
  q.lp[n] = lp;
  if (q.ent) q.ent[n] = ent;
  if (q.lse_out) q.lse_out[n] = lse;
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
  int splits, n_vb, n_tb, group_t, group_s;
  size_t workspace;
};

// One workgroup per CU: split the vocabulary so token blocks x splits fills the machine,
// at least one vocabulary block per split (ranges are spread evenly).
int split_count(int n_tb, int n_vb) {
  const int want = n_tb > 0 ? std::max(1, CU_COUNT / n_tb) : 1;
  return std::max(1, std::min(want, n_vb));
}

// XCD super tiles of 32 workgroups (token blocks x splits) when the grid tiles.
void xcd_groups(Plan* pl) {
  pl->group_t = 0;
  pl->group_s = 0;
  for (int gs : {4, 8, 2, 16, 1, 32}) {
    const int gt = 32 / gs;
    if (pl->splits % gs == 0 && pl->n_tb % gt == 0 && (pl->n_tb * pl->splits) % (8 * 32) == 0) {
      pl->group_t = gt;
      pl->group_s = gs;
      break;
    }
  }
}

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
  pl->splits = split_count(pl->n_tb, pl->n_vb);
  xcd_groups(pl);
  pl->workspace = (size_t)pl->splits * (size_t)d->n_tokens * sizeof(float4);
  return DSV41_OK;
}

// Backward: the forward's grid over the vocabulary range; each workgroup writes the
// logit gradient of every block it sweeps.
int plan_grad(const dsv41_logprob_grad_desc* d, Plan* pl) {
  if (!d) return fail(DSV41_E_INVALID, "log-prob gradient descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_logprob_grad_desc))
    return fail(DSV41_E_ABI, "dsv41_logprob_grad_desc size mismatch (rebuild the binding)");
  if (d->n_tokens < 0 || d->hidden <= 0 || d->vocab <= 0)
    return fail(DSV41_E_INVALID, "hidden states must be [tokens, hidden] and the head [vocab, hidden]");
  if (d->hidden % 8 != 0) return fail(DSV41_E_UNSUPPORTED, "hidden size must be a multiple of 8");
  if (d->x_row_stride < d->hidden || d->w_row_stride < d->hidden || d->x_row_stride % 8 || d->w_row_stride % 8)
    return fail(DSV41_E_INVALID, "row strides must be >= hidden and multiples of 8 elements");
  if (((uintptr_t)d->x | (uintptr_t)d->w | (uintptr_t)d->out) % 16)
    return fail(DSV41_E_INVALID, "hidden states, head weight and output must be 16-byte aligned");
  if ((int64_t)BV * d->w_row_stride * 2 >= (1ll << 31) || (int64_t)BT * d->x_row_stride * 2 >= (1ll << 31))
    return fail(DSV41_E_UNSUPPORTED, "row stride too large for 32-bit block offsets");
  if (!(isfinite(d->temperature) && d->temperature > 0.0f))
    return fail(DSV41_E_INVALID, "temperature must be finite and positive");
  if (!(0 <= d->vocab_begin && d->vocab_begin < d->vocab_end && d->vocab_end <= d->vocab))
    return fail(DSV41_E_INVALID, "vocabulary range must satisfy 0 <= begin < end <= vocab");
  if (d->out_row_stride < d->vocab_end - d->vocab_begin || d->out_row_stride % 8)
    return fail(DSV41_E_INVALID, "output row stride must cover the range and be a multiple of 8 elements");
  if (d->n_tokens > 0 && (!d->x || !d->w || !d->targets || !d->lse || !d->out))
    return fail(DSV41_E_INVALID, "x, w, targets, lse and out are required");
  if (d->grad_entropy && !d->entropy) return fail(DSV41_E_INVALID, "an entropy gradient requires the entropies");
  pl->n_vb = (d->vocab_end - d->vocab_begin + BV - 1) / BV;
  pl->n_tb = (d->n_tokens + BT - 1) / BT;
  pl->splits = split_count(pl->n_tb, pl->n_vb);
  xcd_groups(pl);
  pl->workspace = 0;
  return DSV41_OK;
}

}  // namespace logprob
}  // namespace dsv41

using namespace dsv41;
using namespace dsv41::logprob;

extern "C" int dsv41_logprob_grad_run(const dsv41_logprob_grad_desc* d, void* stream) {
  Plan pl;
  int rc = plan_grad(d, &pl);
  if (rc != DSV41_OK) return rc;
  if (d->n_tokens == 0) return DSV41_OK;
  Params p{};
  p.x = static_cast<const uint16_t*>(d->x);
  p.xs = d->x_row_stride;
  p.ws = d->w_row_stride;
  p.w = static_cast<const uint16_t*>(d->w) + (int64_t)d->vocab_begin * p.ws;
  p.targets = d->targets;
  p.N = d->n_tokens;
  p.H = d->hidden;
  p.V = d->vocab_end - d->vocab_begin;
  p.invT = 1.0f / d->temperature;
  p.splits = pl.splits;
  p.n_vb = pl.n_vb;
  p.n_tb = pl.n_tb;
  p.group_t = pl.group_t;
  p.group_s = pl.group_s;
  p.lse = d->lse;
  p.ent = d->entropy;
  p.glp = d->grad_logprob;
  p.gent = d->grad_entropy;
  p.out = static_cast<uint16_t*>(d->out);
  p.os = d->out_row_stride;
  p.vbeg = d->vocab_begin;
  hipLaunchKernelGGL(fused_kernel<true>, dim3(pl.n_tb * pl.splits), dim3(NT), 0, static_cast<hipStream_t>(stream), p);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}

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
  p.n_vb = pl.n_vb;
  p.n_tb = pl.n_tb;
  p.group_t = pl.group_t;
  p.group_s = pl.group_s;
  hipLaunchKernelGGL(fused_kernel<false>, dim3(pl.n_tb * pl.splits), dim3(NT), 0, s, p);
  DSV41_HIP_CHECK(hipGetLastError());
  MergeParams q{};
  q.part = p.part;
  q.x = p.x;
  q.xs = p.xs;
  q.w = p.w;
  q.ws = p.ws;
  q.targets = d->targets;
  q.N = d->n_tokens;
  q.H = d->hidden;
  q.V = d->vocab;
  q.splits = pl.splits;
  q.invT = p.invT;
  q.behavior = d->behavior;
  q.is_cap = d->is_cap;
  q.lp = d->out_logprob;
  q.ent = d->out_entropy;
  q.ratio = d->out_ratio;
  q.status = d->out_status;
  q.lse_out = d->out_lse;
  hipLaunchKernelGGL(merge_kernel<MERGE_FINAL>, dim3((d->n_tokens + 3) / 4), dim3(256), 0, s, q);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}

// ---------------------------------------------------------------- vocabulary shards
// One GPU's slice of a vocabulary-sharded head: the forward's kernels over the slice, with
// the split states merged into one 16-byte state per token, (max z, sum e, sum e*z, z_t),
// z_t = -inf unless this slice holds the target.  States of all slices, gathered, go to
// dsv41_logprob_combine_run.
namespace {
int shard_plan(const dsv41_logprob_shard_desc* d, dsv41_logprob_desc* fd, Plan* pl) {
  if (!d) return fail(DSV41_E_INVALID, "log-prob shard descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_logprob_shard_desc))
    return fail(DSV41_E_ABI, "dsv41_logprob_shard_desc size mismatch (rebuild the binding)");
  if (d->vocab_offset < 0) return fail(DSV41_E_INVALID, "vocab_offset must be nonnegative");
  if (d->n_tokens > 0 && !d->out_state) return fail(DSV41_E_INVALID, "out_state is required");
  *fd = dsv41_logprob_desc{};
  fd->struct_size = sizeof(dsv41_logprob_desc);
  fd->n_tokens = d->n_tokens;
  fd->hidden = d->hidden;
  fd->vocab = d->vocab;
  fd->x = d->x;
  fd->x_row_stride = d->x_row_stride;
  fd->w = d->w;
  fd->w_row_stride = d->w_row_stride;
  fd->targets = d->targets;
  fd->temperature = d->temperature;
  fd->out_logprob = d->out_state;  // non-null marker for the shared checks
  return plan(fd, pl);
}
}  // namespace

extern "C" size_t dsv41_logprob_shard_workspace_bytes(const dsv41_logprob_shard_desc* d) {
  dsv41_logprob_desc fd;
  Plan pl;
  if (shard_plan(d, &fd, &pl) != DSV41_OK) return 0;
  return pl.workspace;
}

extern "C" int dsv41_logprob_shard_run(const dsv41_logprob_shard_desc* d, void* workspace, size_t workspace_bytes,
                                       void* stream) {
  dsv41_logprob_desc fd;
  Plan pl;
  int rc = shard_plan(d, &fd, &pl);
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
  p.n_vb = pl.n_vb;
  p.n_tb = pl.n_tb;
  p.group_t = pl.group_t;
  p.group_s = pl.group_s;
  hipLaunchKernelGGL(fused_kernel<false>, dim3(pl.n_tb * pl.splits), dim3(NT), 0, s, p);
  DSV41_HIP_CHECK(hipGetLastError());
  MergeParams q{};
  q.part = p.part;
  q.x = p.x;
  q.xs = p.xs;
  q.w = p.w;
  q.ws = p.ws;
  q.targets = d->targets;
  q.N = d->n_tokens;
  q.H = d->hidden;
  q.V = d->vocab;
  q.splits = pl.splits;
  q.voff = d->vocab_offset;
  q.invT = p.invT;
  q.state_out = reinterpret_cast<float4*>(d->out_state);
  hipLaunchKernelGGL(merge_kernel<MERGE_STATE>, dim3((d->n_tokens + 3) / 4), dim3(256), 0, s, q);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}

extern "C" int dsv41_logprob_combine_run(const dsv41_logprob_combine_desc* d, void* stream) {
  if (!d) return fail(DSV41_E_INVALID, "log-prob combine descriptor is NULL");
  if (d->struct_size != sizeof(dsv41_logprob_combine_desc))
    return fail(DSV41_E_ABI, "dsv41_logprob_combine_desc size mismatch (rebuild the binding)");
  if (d->n_tokens < 0 || d->n_shards <= 0) return fail(DSV41_E_INVALID, "need at least one shard and n_tokens >= 0");
  if (d->n_tokens > 0 && (!d->states || !d->out_logprob))
    return fail(DSV41_E_INVALID, "states and out_logprob are required");
  if (((uintptr_t)d->states) % 16) return fail(DSV41_E_INVALID, "states must be 16-byte aligned");
  if (d->out_ratio && !d->behavior) return fail(DSV41_E_INVALID, "ratio output requires behavior log-probs");
  if (d->behavior && !(isfinite(d->is_cap) && d->is_cap > 0.0f))
    return fail(DSV41_E_INVALID, "is_cap must be finite and positive");
  if (d->n_tokens == 0) return DSV41_OK;
  MergeParams q{};
  q.part = reinterpret_cast<const float4*>(d->states);
  q.N = d->n_tokens;
  q.splits = d->n_shards;
  q.behavior = d->behavior;
  q.is_cap = d->is_cap;
  q.lp = d->out_logprob;
  q.ent = d->out_entropy;
  q.ratio = d->out_ratio;
  q.status = d->out_status;
  q.lse_out = d->out_lse;
  hipLaunchKernelGGL(merge_kernel<MERGE_COMBINE>, dim3((d->n_tokens + 3) / 4), dim3(256), 0,
                     static_cast<hipStream_t>(stream), q);
  DSV41_HIP_CHECK(hipGetLastError());
  return DSV41_OK;
}
