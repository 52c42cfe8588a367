// Speculative-decoding verifier and token sampler over the full vocabulary (replaces verify_drafts and
// Sampler.forward, nanovllm/layers/sampler.py:5-103).
//
// Two HBM-streaming kernels over [rows, vocab] tables and a small one between them. A row is cut into at most kSpans
// contiguous spans (a multiple of 4 entries each, none empty); a 256-thread workgroup streams one span with
// 4-entry loads (16 B for fp32, 8 B for bf16; scalar loads when the rows are not aligned).
//   1. row_stats       (row, span): first argmax of the raw logits of target rows; for rows with temperature
//                      != 0 also max and sum(exp(x - max)) of x = l / T (target rows and, when given, draft
//                      rows), kept per thread online and combined in a fixed order.
//   verify_decide      (seq): merges span stats in span order (argmax, logsumexp), applies the accept rule
//                      u * q(d) < p(d) (or top1 == d for greedy rows) to the leading run of real guesses,
//                      writes num_accepted, for greedy rows next_token, and the sequence's decision for the
//                      resample. (Taking the decision in the prologue of every resample workgroup instead
//                      cost as much as this launch: the resample's loads then wait for it.)
//   2. verify_resample (seq, span): random rows only, over up to 64 spans per row (a single row per
//                      sequence: more spans keep a small batch spread over the GPU): the first argmax of
//                      p / max(E, 1e-10) and of residual / max(E, 1e-10) with p = softmax(row a / T), residual =
//                      max(p - q, 0) (or p with the rejected n-gram guess zeroed), and whether any residual is
//                      positive; exact values only for the entries that bounds cannot rule out.
//                      The last of a sequence's resample workgroups (an arrival count per sequence, zeroed
//                      by verify_decide; the candidates written and read with the agent-scope cache bit)
//                      merges the span candidates and picks the token: no launch of its own.
// Every reduction has a fixed order, so results are deterministic; ties resolve to the first index (and a
// NaN counts as the largest value), as torch.argmax does.
#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "lm_head.h"
#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {
namespace {

constexpr int kSpans = 6;         // most spans per row (workgroups per row; 6 measured best of 4 / 6 / 8 / 12 / 16)
constexpr int kPipeU = 2;         // verify_resample: 4-entry groups a lane loads per pipeline stage
constexpr int kThreads = 256;

struct RowStat {                  // per (row, chunk)
  float max_x;                    // max of l / T over the chunk (random rows; -inf for an all -inf chunk)
  float sum;                      // sum of exp(l / T - lse_shift(max_x)) (random rows)
  float best;                     // raw logit at the chunk's first argmax (greedy target rows)
  int32_t best_idx;
};

struct SeqInfo {
  int32_t a;                      // accepted guesses
  int32_t random;                 // 1 if temperature != 0
  int32_t resid_mode;             // 0: sample from p; 1: n-gram (zero the guess if rejected); 2: draft residual
  int32_t rejected;               // a < num_drafts
  int32_t guess;                  // guess token of the rejected slot (n-gram), or -1
  float Ma, Sa;                   // softmax of target row a: shift lse_shift(max) and sum of exp(x - shift)
  float Md, Sd;                   // the same for the draft row of the rejected slot
  float pad[3];
};

struct Cand {                     // per (seq, chunk)
  float p_val;
  int32_t p_idx;
  float r_val;
  int32_t r_idx;
  int32_t any_res;
  int32_t pad[3];
};

template <int DT>
__device__ __forceinline__ float load_logit(const void* base, int64_t idx) {
  if (DT == SD_DTYPE_F32) return ((const float*)base)[idx];
  return bf16_bits_to_f32(((const uint16_t*)base)[idx]);
}

// Entries idx .. idx+3 (idx a multiple of 4; the row 16-byte aligned for fp32, 8-byte for bf16).
template <int DT>
__device__ __forceinline__ float4 load_logit4(const void* base, int64_t idx) {
  if (DT == SD_DTYPE_F32) return *(const float4*)((const float*)base + idx);
  const uint2 w = *(const uint2*)((const uint16_t*)base + idx);
  return make_float4(__builtin_bit_cast(float, w.x << 16), __builtin_bit_cast(float, w.x & 0xffff0000u),
                     __builtin_bit_cast(float, w.y << 16), __builtin_bit_cast(float, w.y & 0xffff0000u));
}

// exp(x) to about 1.5 ulp, for every exponential of the sampler: x*log2(e) is split into an integer n and a
// fraction f, the product's rounding error carried into f by two fma (log2(e) as a pair of floats), then
// 2^f from v_exp_f32 (1 ulp on [-0.5, 0.5]) scaled by 2^n. Inputs are clamped to [-110, 100], where exp
// already rounds to 0 or overflows to inf (NaN stays NaN).
// Contraction is off here: fusing the product t into (t - n) would count its rounding error twice.
__device__ __forceinline__ float exp_acc(float x) {
#pragma clang fp contract(off)
  x = x < -110.f ? -110.f : (x > 100.f ? 100.f : x);
  const float kHi = 1.44269502162933349609375f;   // log2(e) rounded to fp32
  const float kLo = 1.925963033500011e-08f;       // log2(e) - kHi
  const float t = x * kHi;
  const float n = __builtin_rintf(t);
  const float f = (t - n) + fmaf(x, kLo, fmaf(x, kHi, -t));
  return ldexpf(__builtin_amdgcn_exp2f(f), (int)n);
}

// exp(x) for the terms of the streaming sums: v_exp_f32 (0.77 ulp over its whole range) of the rounded
// product t = x*log2(e), corrected by that product's rounding error with one fma: within 1.25 ulp of e^x for
// normal results (measured on 4M inputs in [-120, 5]); results below 2^-126 flush to 0, which no sum that holds
// a term exp(0) = 1 can see. x = -inf gives 0 (clamped to -104 first), NaN stays NaN.
__device__ __forceinline__ float exp_term(float x) {
#pragma clang fp contract(off)
  x = x < -104.f ? -104.f : x;
  const float kHi = 1.44269502162933349609375f;
  const float kLo = 1.925963033500011e-08f;
  const float t = x * kHi;
  const float err = fmaf(x, kLo, fmaf(x, kHi, -t));
  const float r = __builtin_amdgcn_exp2f(t);
  return fmaf(r, err * 0.693147180559945309f, r);
}

// x / T with z = 1/T correctly rounded (one division per workgroup): y = x*z lies within an ulp of the
// quotient, its residual x - y*T is exact (fma), and one correction step gives the correctly rounded quotient
// (Markstein's theorem; checked against IEEE division on 2.8e9 random fp32 x in [2^-100, 2^100] for 18
// temperatures from 0.01 to 3). Infinite x keeps its sign; tiny x may be an ulp off, which no sum of
// exponentials sees. Used by the streaming passes only; the decisions divide.
__device__ __forceinline__ float div_by(float x, float T, float z) {
#pragma clang fp contract(off)
  const float y = x * z;
  return __builtin_isinf(y) ? y : fmaf(fmaf(-y, T, x), z, y);
}

// The shift of a logsumexp: the maximum, or 0 when it is infinite (torch.logsumexp's rule), so that
// an all -inf set sums to 0 (lse -inf) and a +inf entry gives +inf.
__device__ __forceinline__ float lse_shift(float m) { return fabsf(m) == INFINITY ? 0.f : m; }

// Online (max m, sum s of exp(x - lse_shift(m))) of one thread's entries. s == 0 exactly while every entry
// seen is -inf; a rescale leaves it 0 then (it would multiply 0 by an overflowing factor). A +inf entry makes
// the sum +inf (finish()).
struct OnlineSum {
  float m = -INFINITY, s = 0.f;
  // Adds N entries: one rescale to their common max, then N exponentials.
  template <int N>
  __device__ __forceinline__ void add(const float (&x)[N]) {
    float ml = x[0];
#pragma unroll
    for (int e = 1; e < N; ++e) ml = fmaxf(ml, x[e]);
    const float mn = fmaxf(m, ml);
    const float f = exp_term(lse_shift(m) - lse_shift(mn));
    s = s != 0.f ? s * f : 0.f;
    m = mn;
    const float sh = lse_shift(m);
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < N; ++e) acc += exp_term(x[e] - sh);
    s += acc;
  }
  __device__ __forceinline__ void finish() {
    if (m == INFINITY) s = INFINITY;
  }
};

// (m, s) of two disjoint sets merged: the sum rescaled to the larger max; an empty side (s == 0) adds 0.
__device__ __forceinline__ void merge_pair(float& m, float& s, float om, float os) {
  const float M = fmaxf(m, om);
  const float shM = lse_shift(M);
  s = (s != 0.f ? s * exp_acc(lse_shift(m) - shM) : 0.f) + (os != 0.f ? os * exp_acc(lse_shift(om) - shM) : 0.f);
  m = M;
}

// Block-wide reductions over 256 threads (4 waves) in a fixed order.
__device__ __forceinline__ float block_max(float v, float* sh) {
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (threadIdx.x % kWave == 0) sh[w] = v;
  __syncthreads();
  return fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
}

__device__ __forceinline__ float block_sum(float v, float* sh) {
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (threadIdx.x % kWave == 0) sh[w] = v;
  __syncthreads();
  return ((sh[0] + sh[1]) + sh[2]) + sh[3];
}

// Combines the threads' (max, sum) pairs in a fixed order: lanes by xor-shuffle, then waves 0..3.
__device__ __forceinline__ void combine_online(OnlineSum& o, float* sh) {
  for (int off = 32; off >= 1; off >>= 1) {
    const float om = __shfl_xor(o.m, off), os = __shfl_xor(o.s, off);
    merge_pair(o.m, o.s, om, os);
  }
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (threadIdx.x % kWave == 0) {
    sh[2 * w] = o.m;
    sh[2 * w + 1] = o.s;
  }
  __syncthreads();
  float M = sh[0], S = sh[1];
  for (int k = 1; k < 4; ++k) merge_pair(M, S, sh[2 * k], sh[2 * k + 1]);
  o.m = M;
  o.s = S;
}

__device__ __forceinline__ void block_argmax(float& v, int& i, float* shv, int* shi) {
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int oi = __shfl_xor(i, off);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
  const int w = threadIdx.x / kWave;
  __syncthreads();
  if (threadIdx.x % kWave == 0) {
    shv[w] = v;
    shi[w] = i;
  }
  __syncthreads();
  v = shv[0];
  i = shi[0];
  for (int k = 1; k < 4; ++k)
    if (better(shv[k], shi[k], v, i)) {
      v = shv[k];
      i = shi[k];
    }
}

struct VParams {
  const void* logits;
  int64_t logits_stride;
  const int64_t* drafts;          // [S, K]
  const int64_t* num_drafts;      // [S]
  const float* temps;             // [S], or null: every row greedy
  const void* draft_logits;       // [S*K] rows or null
  int64_t draft_stride;
  const float* uniforms;          // [S, K]
  const float* noise;             // [S, V]
  int32_t S, K, V, nchunk, span;  // row_stats: nchunk spans of `span` entries (the last may be shorter)
  int32_t rchunk, rspan;          // verify_resample: rchunk spans of `rspan` entries
  int64_t* out_a;
  int64_t* out_next;
  RowStat* stats;                 // [(S*(K+1) + S*K) rows][nchunk]
  SeqInfo* info;                  // [S]
  Cand* cand;                     // [S][rchunk]
  int32_t* done;                  // [S]: verify_resample's arrival counters, zeroed by verify_decide (sampled calls)
};

// One span of one row: the first argmax of the raw values (kArg) and the online (max, sum) of x = value / T
// (kSum; kDiv when T != 1). A thread visits v0 + 4*tid, then every 4*kThreads entries, in increasing order;
// the aligned main loop has four of those 4-entry loads in flight and folds their 16 entries into the sum with
// one rescale. Within a thread indices only grow, so a later entry replaces the argmax only when larger (or
// NaN over a non-NaN), which is torch.argmax's first-index rule.
template <int DTX, bool kVec, bool kArg, bool kSum, bool kDiv>
__device__ __forceinline__ void scan_span(const void* base, int v0, int v1, float T, float z, float& bv, int& bi,
                                          OnlineSum& os) {
  auto arg = [&](float r, int v) {
    if (bv == bv && !(r <= bv)) {
      bv = r;
      bi = v;
    }
  };
  auto xof = [&](float r) { return kDiv ? div_by(r, T, z) : r; };
  constexpr int kStep = 4 * kThreads;
  int v = v0 + 4 * threadIdx.x;
  if (kVec) {
    for (; v + 3 * kStep + 4 <= v1; v += 4 * kStep) {
      float4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = load_logit4<DTX>(base, v + u * kStep);
      float x[16];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float r[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (kArg) arg(r[e], v + u * kStep + e);
          x[4 * u + e] = xof(r[e]);
        }
      }
      if (kSum) os.add(x);
    }
  }
  for (; v < v1; v += kStep) {
    float r[4];
    if (kVec && v + 4 <= v1) {
      const float4 q4 = load_logit4<DTX>(base, v);
      r[0] = q4.x, r[1] = q4.y, r[2] = q4.z, r[3] = q4.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = v + e < v1 ? load_logit<DTX>(base, v + e) : -INFINITY;
    }
    float x[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (kArg && v + e < v1) arg(r[e], v + e);
      x[e] = v + e < v1 ? xof(r[e]) : -INFINITY;
    }
    if (kSum) os.add(x);
  }
}

// Grid (rows, spans): target rows first (argmax; with a temperature also the softmax statistics of l / T),
// then the draft rows of sampled sequences (statistics only). Each workgroup takes one uniform branch to the
// scan it needs.
template <int DT, int DDT, bool kVec, bool kRand>
__global__ __launch_bounds__(kThreads) void row_stats(VParams p) {
  __shared__ float shf[8];
  __shared__ int shi[4];
  const int row = blockIdx.x;
  const int chunk = blockIdx.y;
  const int target_rows = p.S * (p.K + 1);
  const bool is_target = row < target_rows;
  const int seq = is_target ? row / (p.K + 1) : (row - target_rows) / p.K;
  const float T = kRand ? p.temps[seq] : 0.f;
  const bool random = kRand && T != 0.f;
  if (!is_target && !random) return;  // draft rows only matter for sampled rows
  const int v0 = chunk * p.span;
  const int v1 = min(v0 + p.span, p.V);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  OnlineSum os;
  const float z = random ? 1.f / T : 1.f;
  if (is_target) {
    // The first argmax matters for greedy rows only (the decision and the next token of a sampled row use
    // the softmax statistics and the noise): sampled rows skip it.
    const void* base = DT == SD_DTYPE_F32
                           ? (const void*)((const float*)p.logits + (int64_t)row * p.logits_stride)
                           : (const void*)((const uint16_t*)p.logits + (int64_t)row * p.logits_stride);
    if (!random)
      scan_span<DT, kVec, true, false, false>(base, v0, v1, T, z, bv, bi, os);
    else if (T == 1.f)
      scan_span<DT, kVec, false, true, false>(base, v0, v1, T, z, bv, bi, os);
    else
      scan_span<DT, kVec, false, true, true>(base, v0, v1, T, z, bv, bi, os);
  } else {
    const int64_t dr = row - target_rows;
    const void* base = DDT == SD_DTYPE_F32 ? (const void*)((const float*)p.draft_logits + dr * p.draft_stride)
                                           : (const void*)((const uint16_t*)p.draft_logits + dr * p.draft_stride);
    if (T == 1.f)
      scan_span<DDT, kVec, false, true, false>(base, v0, v1, T, z, bv, bi, os);
    else
      scan_span<DDT, kVec, false, true, true>(base, v0, v1, T, z, bv, bi, os);
  }
  RowStat st;
  st.max_x = -INFINITY;
  st.sum = 0.f;
  if (is_target && !random) block_argmax(bv, bi, shf, shi);
  st.best = bv;
  st.best_idx = bi;
  if (random) {
    os.finish();
    combine_online(os, shf);
    st.max_x = os.m;
    st.sum = os.s;
  }
  if (threadIdx.x == 0) p.stats[(int64_t)row * p.nchunk + chunk] = st;
}

// A row's softmax statistics from its chunks, in chunk order: the shift lse_shift(max over chunks) and
// sum = sum_c sum_c * exp(lse_shift(max_c) - shift); chunks whose entries are all -inf (sum 0) add nothing.
// logsumexp = log(sum) + shift (-inf for an all -inf row).
__device__ void merge_softmax(const RowStat* st, int nchunk, float* shift_out, float* S_out) {
  float M = -INFINITY;
  for (int c = 0; c < nchunk; ++c) M = fmaxf(M, st[c].max_x);
  const float shM = lse_shift(M);
  float s = 0.f;
  for (int c = 0; c < nchunk; ++c)
    if (st[c].sum != 0.f) s += st[c].sum * exp_acc(lse_shift(st[c].max_x) - shM);
  *shift_out = shM;
  *S_out = s;
}

// The decision for one sequence, by one workgroup of 64 threads. Every global read is issued up front (the
// span statistics of the sequence's rows into LDS; per guess slot the guess, its uniform and its target and
// draft logits), then lane j merges row j's spans and evaluates guess j, and the leading run of accepts gives
// a. Thread 0 writes num_accepted, the greedy token and the sequence's SeqInfo.
template <int DT, int DDT, bool kRand>
__global__ __launch_bounds__(64) void verify_decide(VParams p) {
  const int seq = blockIdx.x;
  __shared__ RowStat sst[(64 + 63) * kSpans];
  __shared__ int32_t top1[64];
  __shared__ float lse[64], dlse[64], tshift[64], tsum[64], dshift[64], dsum[64];
  __shared__ int accj[64];
  __shared__ int64_t guess[64];
  const int lane = threadIdx.x;
  const int nthr = blockDim.x;
  const int K = p.K, nchunk = p.nchunk;
  const float T = kRand ? p.temps[seq] : 0.f;
  const bool random = kRand && T != 0.f;
  const bool draft = random && p.draft_logits;
  const int target_rows = p.S * (K + 1);
  const int nt = (K + 1) * nchunk, nd_stats = draft ? K * nchunk : 0;
  const RowStat* tst = p.stats + (int64_t)seq * (K + 1) * nchunk;
  const RowStat* dst = p.stats + ((int64_t)target_rows + (int64_t)seq * K) * nchunk;
  for (int i = lane; i < nt; i += nthr) sst[i] = tst[i];
  for (int i = lane; i < nd_stats; i += nthr) sst[nt + i] = dst[i];
  const int64_t nd = p.num_drafts ? p.num_drafts[seq] : 0;
  int64_t d = -1;
  float xl = 0.f, xd = 0.f, u = 1.f;
  if (lane < K) {
    d = guess[lane] = p.drafts[(int64_t)seq * K + lane];
    if (random && d >= 0 && d < p.V) {
      const int64_t trow = (int64_t)seq * (K + 1) + lane;
      xl = DT == SD_DTYPE_F32 ? ((const float*)p.logits)[trow * p.logits_stride + d]
                              : bf16_bits_to_f32(((const uint16_t*)p.logits)[trow * p.logits_stride + d]);
      if (draft) {
        const int64_t dr = (int64_t)seq * K + lane;
        xd = DDT == SD_DTYPE_F32 ? ((const float*)p.draft_logits)[dr * p.draft_stride + d]
                                 : bf16_bits_to_f32(((const uint16_t*)p.draft_logits)[dr * p.draft_stride + d]);
      }
      if (p.uniforms) u = p.uniforms[(int64_t)seq * K + lane];  // missing uniforms: u = 1
    }
  }
  __syncthreads();
  if (lane <= K) {
    const RowStat* st = sst + lane * nchunk;
    float bv = st[0].best;
    int bi = st[0].best_idx;
    for (int c = 1; c < nchunk; ++c)
      if (better(st[c].best, st[c].best_idx, bv, bi)) {
        bv = st[c].best;
        bi = st[c].best_idx;
      }
    top1[lane] = bi;
    if (random) {
      merge_softmax(st, nchunk, &tshift[lane], &tsum[lane]);
      lse[lane] = logf(tsum[lane]) + tshift[lane];
    }
  }
  if (draft && lane < K) {
    merge_softmax(sst + nt + lane * nchunk, nchunk, &dshift[lane], &dsum[lane]);
    dlse[lane] = logf(dsum[lane]) + dshift[lane];
  }
  __syncthreads();
  if (lane < K) {
    bool acc = false;
    if (lane < nd && d >= 0 && d < p.V) {
      if (!random) {
        acc = top1[lane] == d;
      } else {
        const float pd = exp_acc(xl / T - lse[lane]);
        const float qd = draft ? exp_acc(xd / T - dlse[lane]) : 1.f;
        acc = u * qd < pd;
      }
    }
    accj[lane] = acc ? 1 : 0;
  }
  __syncthreads();
  if (lane == 0) {
    int a = 0;
    while (a < K && accj[a]) ++a;
    SeqInfo info{};
    info.a = a;
    info.random = random ? 1 : 0;
    info.guess = -1;
    if (random) {
      info.Ma = tshift[a];
      info.Sa = tsum[a];
      info.rejected = a < nd ? 1 : 0;
      if (K > 0) {
        const int j = min(a, K - 1);
        if (draft) {
          info.resid_mode = 2;
          info.Md = dshift[j];
          info.Sd = dsum[j];
        } else {
          info.resid_mode = 1;
          const int64_t dj = guess[j];
          info.guess = (dj >= 0 && dj < p.V) ? (int32_t)dj : -1;
        }
      }
    }
    p.out_a[seq] = a;
    if (!random) p.out_next[seq] = top1[a];
    p.info[seq] = info;
    if (kRand && p.done) p.done[seq] = 0;
  }
}

// A resample span's candidate, written and read with the agent-scope cache bit (the bit the memory model
// gives agent-scope atomic stores and loads): coherent across the XCDs' L2s without a fence that writes back
// or invalidates a whole L2.
__device__ __forceinline__ void store_cand(Cand* dst, const Cand& c) {
  __hip_atomic_store((int32_t*)&dst->p_val, __float_as_int(c.p_val), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&dst->p_idx, c.p_idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store((int32_t*)&dst->r_val, __float_as_int(c.r_val), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&dst->r_idx, c.r_idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(&dst->any_res, c.any_res, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ Cand load_cand(const Cand* src) {
  Cand c{};
  c.p_val = __int_as_float(__hip_atomic_load((const int32_t*)&src->p_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  c.p_idx = __hip_atomic_load(&src->p_idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c.r_val = __int_as_float(__hip_atomic_load((const int32_t*)&src->r_val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
  c.r_idx = __hip_atomic_load(&src->r_idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  c.any_res = __hip_atomic_load(&src->any_res, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return c;
}

// The sampled token of a random sequence, by the last of its resample workgroups: thread k reads span k's
// candidate (all reads in flight together), then the same block reductions as inside a span. The argmax
// order (value, then lower index) makes the result independent of the reduction tree.
__device__ __forceinline__ void finish_seq(const VParams& p, int seq, const SeqInfo& info, float* shf, int* shi) {
  float pv = -INFINITY, rv = -INFINITY;
  int pi = 0x7fffffff, ri = 0x7fffffff, any_res = 0;
  for (int k = threadIdx.x; k < p.rchunk; k += kThreads) {
    const Cand c = load_cand(p.cand + (int64_t)seq * p.rchunk + k);
    if (better(c.p_val, c.p_idx, pv, pi)) {
      pv = c.p_val;
      pi = c.p_idx;
    }
    if (better(c.r_val, c.r_idx, rv, ri)) {
      rv = c.r_val;
      ri = c.r_idx;
    }
    any_res |= c.any_res;
  }
  block_argmax(pv, pi, shf, shi);
  block_argmax(rv, ri, shf, shi);
  any_res = __syncthreads_or(any_res);
  const bool use_res = info.resid_mode == 2 && info.rejected && any_res;
  if (threadIdx.x == 0) p.out_next[seq] = use_res ? ri : pi;
}

// verify_resample streams its span with approximate values and computes exact ones only where they can matter.
// The exact values are the reference's: prob = exp(x - shift) / sum with x = l / T, p / max(E, 1e-10) and
// max(prob - q, 0) / max(E, 1e-10), each an IEEE division of exp_acc results. The approximations replace the
// divisions by products with reciprocals and the exponential by one v_exp_f32; for every entry whose prob is a
// normal number they are within eps = (|shift| + 323) * 2^-22 of the exact values (x = l / T within 1.5 * 2^-23 |x|,
// the subtraction and the product with log2(e) 2^-24 of |x - shift| each, v_exp_f32 1 ulp, reciprocals and
// products a few ulps; |x - shift| <= 104.5 wherever exp_acc does not underflow to 0). So each entry has a lower
// bound lb <= exact <= ub, and with L the largest lower bound of the span, the winner (and every entry tied with
// it) has ub >= L. A lane keeps the entry with the largest ub and the second-largest ub; when that second is below
// L, its only entry that can reach L is the first, which is computed exactly. Otherwise (and whenever the bounds
// are not trusted: L below 2^-60, where flushed approximations of exact values up to 2^-126 / 1e-10 may hide, a
// NaN, or no residual sure to be positive) the lane reads its entries again and computes exactly each one that
// may reach L (every one with a possibly non-zero prob in the untrusted cases). The exact argmax (ties: the
// lower index) of the computed entries is then the argmax over all entries.
constexpr float kTinyBest = 8.673617379884035e-19f;  // 2^-60
constexpr float kUnderflow = -104.5f;

template <int DT, int DDT, bool kVec>
__global__ __launch_bounds__(kThreads) void verify_resample(VParams p) {
  __shared__ float shf[8];
  __shared__ int shi[4];
  const int seq = blockIdx.x;
  const int chunk = blockIdx.y;
  const float T = p.temps[seq];
  const SeqInfo info = p.info[seq];  // verify_decide's
  if (!info.random) return;
  const bool div = T != 1.f;
  const float z = 1.f / T;
  const int K = p.K;
  const int64_t trow = (int64_t)seq * (K + 1) + info.a;
  const int64_t drow = (int64_t)seq * K + min(info.a, K - 1);
  const void* tbase = DT == SD_DTYPE_F32 ? (const void*)((const float*)p.logits + trow * p.logits_stride)
                                         : (const void*)((const uint16_t*)p.logits + trow * p.logits_stride);
  const bool resid = info.resid_mode == 2;
  const void* dbase = nullptr;
  if (resid)
    dbase = DDT == SD_DTYPE_F32 ? (const void*)((const float*)p.draft_logits + drow * p.draft_stride)
                                : (const void*)((const uint16_t*)p.draft_logits + drow * p.draft_stride);
  const float* noise = p.noise ? p.noise + (int64_t)seq * p.V : nullptr;  // missing noise: E = 1
  const int zap = info.resid_mode == 1 && info.rejected ? info.guess : -1;  // n-gram: prob of the guess is 0
  const float kL2E = 1.4426950408889634f;
  const float eps = (fmaxf(fabsf(info.Ma), resid ? fabsf(info.Md) : 0.f) + 323.f) * 2.384185791015625e-07f;
  const float up = 1.f + 2.f * eps, dn = 1.f - 2.f * eps;
  const int v0 = chunk * p.rspan;
  const int v1 = min(v0 + p.rspan, p.V);
  float pv = -INFINITY, rv = -INFINITY;
  int pi = 0x7fffffff, ri = 0x7fffffff;
  int any_res = 0;
  // Exact values of entry i, folded into the lane's bests.
  auto exact = [&](int i, float l, float E, float ld) {
    float prob = exp_acc((div ? l / T : l) - info.Ma) / info.Sa;
    const float Ee = noise ? fmaxf(E, 1e-10f) : 1.f;
    if (i == zap) prob = 0.f;
    const float sp = prob / Ee;
    if (better(sp, i, pv, pi)) {
      pv = sp;
      pi = i;
    }
    if (resid) {
      const float q = exp_acc((div ? ld / T : ld) - info.Md) / info.Sd;
      const float res = fmaxf(prob - q, 0.f);
      any_res |= res > 0.f;
      const float sr = res / Ee;
      if (better(sr, i, rv, ri)) {
        rv = sr;
        ri = i;
      }
    }
  };
  auto reload = [&](int i) {
    exact(i, load_logit<DT>(tbase, i), noise ? noise[i] : 1.f, dbase ? load_logit<DDT>(dbase, i) : 0.f);
  };
  // Upper bounds of entry i (of p / E and of the residual), a lower bound of its residual, whether its prob may
  // be non-zero and whether its residual is surely positive. The lower bound of p / E is ubp * dn / up.
  // log2(1 / sum) is folded into the exponent (one fma): sum <= vocab < 2^31, so it adds at most 31 * 2^-23
  // (v_log_f32, 1 ulp) and 2^-24 (|x - shift| + 31) (the fma), which eps covers.
  const float lsa = -__builtin_log2f(info.Sa), lsd = resid ? -__builtin_log2f(info.Sd) : 0.f;
  struct Bounds {
    float ubp, ubr, lbr;
    bool live, sure;
  };
  // Specialised by mode (residual or not, division by T or not), so that the first pass has no per-entry
  // branch; with noise absent E is 1 and max(E, 1e-10) is 1.
  auto bounds_t = [&](auto resid_c, auto div_c, int i, float l, float E, float ld) {
#pragma clang fp contract(off)
    constexpr bool kR = decltype(resid_c)::value, kD = decltype(div_c)::value;
    Bounds b;
    const float rE = __builtin_amdgcn_rcpf(fmaxf(E, 1e-10f));
    const float dp = (kD ? l * z : l) - info.Ma;
    const float pa = !kR && i == zap ? 0.f : exp2_fast(fmaf(dp, kL2E, lsa));  // zap is -1 in residual mode
    b.live = dp > kUnderflow;
    b.ubp = pa * rE * up;
    b.ubr = b.lbr = 0.f;
    b.sure = false;
    if constexpr (kR) {
      const float qa = exp2_fast(fmaf((kD ? ld * z : ld) - info.Md, kL2E, lsd));
      const float slack = 2.f * eps * (pa + qa);
      b.ubr = (fmaxf(pa - qa, 0.f) + slack) * rE * up;
      b.lbr = fmaxf(pa - qa - slack, 0.f) * rE * dn;
      b.sure = pa - qa - slack > 0.f;
    }
    return b;
  };
  using True_ = std::true_type;
  using False_ = std::false_type;
  auto bounds = [&](int i, float l, float E, float ld) {
    if (resid) return div ? bounds_t(True_{}, True_{}, i, l, E, ld) : bounds_t(True_{}, False_{}, i, l, E, ld);
    return div ? bounds_t(False_{}, True_{}, i, l, E, ld) : bounds_t(False_{}, False_{}, i, l, E, ld);
  };
  // Pass over the span, in rounds of 8 entries a lane (v .. v+3 and v+kStep .. v+kStep+3).
  constexpr int kStep = 4 * kThreads;
  const int rounds = (v1 - v0 + 2 * kStep - 1) / (2 * kStep);
  auto sweep = [&](auto&& visit) {
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int v = v0 + r * 2 * kStep + u * kStep + 4 * threadIdx.x;
        if (kVec && v + 4 <= v1) {
          const float4 t4 = load_logit4<DT>(tbase, v);
          const float4 e4 = noise ? *(const float4*)(noise + v) : make_float4(1.f, 1.f, 1.f, 1.f);
          const float4 d4 = dbase ? load_logit4<DDT>(dbase, v) : make_float4(0.f, 0.f, 0.f, 0.f);
          visit(v, t4.x, e4.x, d4.x);
          visit(v + 1, t4.y, e4.y, d4.y);
          visit(v + 2, t4.z, e4.z, d4.z);
          visit(v + 3, t4.w, e4.w, d4.w);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (v + e < v1)
              visit(v + e, load_logit<DT>(tbase, v + e), noise ? noise[v + e] : 1.f,
                    dbase ? load_logit<DDT>(dbase, v + e) : 0.f);
        }
      }
    }
  };
  // Per lane: the entry with the largest upper bound and the second-largest upper bound (the entry's values
  // are read again for its exact evaluation).
  float b1p = -INFINITY, b2p = -INFINITY, b1r = -INFINITY, b2r = -INFINITY, lr = -INFINITY;
  int i1p = -1, i1r = -1;
  bool sure = false, odd = false;
  // Branch-free updates (selects, which keep the running value where an entry is NaN, as fmaxf does): early
  // in the span nearly every entry is some lane's new best, so a branch would run the update code for the
  // whole wave anyway. One instantiation per mode.
  // The first pass over aligned rows with noise, software-pipelined: the loads of a lane's next kPipeU groups
  // of 4 entries are in flight while the current ones are screened (two register buffers, used in turn, so
  // that no copy waits for loads). Aligned noise rows make the vocabulary a multiple of 4, so a span is whole
  // 4-entry groups; addresses past the span's end are clamped to its last group and those entries skipped.
  struct Stage {
    float4 t[kPipeU], e[kPipeU], d[kPipeU];
  };
  constexpr int kStage = kPipeU * kStep;
  const int stages = (v1 - v0 + kStage - 1) / kStage;
  auto pipe = [&](auto resid_c, auto&& visit) {
    constexpr bool kR = decltype(resid_c)::value;
    auto load = [&](int g, Stage& st) {
#pragma unroll
      for (int u = 0; u < kPipeU; ++u) {
        const int v = min(v0 + g * kStage + u * kStep + 4 * (int)threadIdx.x, v1 - 4);
        st.t[u] = load_logit4<DT>(tbase, v);
        st.e[u] = *(const float4*)(noise + v);
        if (kR) st.d[u] = load_logit4<DDT>(dbase, v);
      }
    };
    auto run = [&](int g, const Stage& st) {
#pragma unroll
      for (int u = 0; u < kPipeU; ++u) {
        const int v = v0 + g * kStage + u * kStep + 4 * threadIdx.x;
        if (v < v1) {
          const float4 d4 = kR ? st.d[u] : make_float4(0.f, 0.f, 0.f, 0.f);
          visit(v, st.t[u].x, st.e[u].x, d4.x);
          visit(v + 1, st.t[u].y, st.e[u].y, d4.y);
          visit(v + 2, st.t[u].z, st.e[u].z, d4.z);
          visit(v + 3, st.t[u].w, st.e[u].w, d4.w);
        }
      }
    };
    Stage a, b;
    load(0, a);
    for (int g = 0; g < stages; g += 2) {
      load(g + 1, b);
      run(g, a);
      load(g + 2, a);
      run(g + 1, b);
    }
  };
  auto first_pass = [&](auto resid_c, auto div_c) {
    constexpr bool kR = decltype(resid_c)::value;
    auto scan = [&](auto&& visit) {
      if constexpr (kVec) {
        if (noise) return pipe(resid_c, visit);
      }
      sweep(visit);
    };
    scan([&](int i, float l, float E, float ld) {
      const Bounds b = bounds_t(resid_c, div_c, i, l, E, ld);
      odd = odd || b.ubp != b.ubp || (kR && b.ubr != b.ubr);
      const bool np = b.ubp > b1p;
      b2p = np ? b1p : (b.ubp > b2p ? b.ubp : b2p);
      i1p = np ? i : i1p;
      b1p = np ? b.ubp : b1p;
      if constexpr (kR) {
        const bool nr = b.ubr > b1r;
        b2r = nr ? b1r : (b.ubr > b2r ? b.ubr : b2r);
        i1r = nr ? i : i1r;
        b1r = nr ? b.ubr : b1r;
        lr = b.lbr > lr ? b.lbr : lr;
        sure = sure || b.sure;
      }
    });
  };
  if (resid) {
    if (div) first_pass(True_{}, True_{}); else first_pass(True_{}, False_{});
  } else {
    if (div) first_pass(False_{}, True_{}); else first_pass(False_{}, False_{});
  }
  // The largest lower bound of p / E in the span: the largest upper bound scaled down, less one rounding.
  const float Lp = block_max(b1p, shf) * (dn / up) * (1.f - 2.384185791015625e-07f);
  const float Lr = resid ? block_max(lr, shf + 4) : 0.f;
  const bool sure_any = resid && __syncthreads_or(sure);
  const bool tiny_p = !(Lp >= kTinyBest), tiny_r = resid && !(Lr >= kTinyBest);
  if (sure) any_res = 1;
  const bool rescan = odd || tiny_p || tiny_r || (resid && !sure_any) || b2p >= Lp || (resid && b2r >= Lr);
  if (!rescan) {
    const bool ep = i1p >= 0 && b1p >= Lp;
    if (ep) reload(i1p);
    if (resid && i1r >= 0 && b1r >= Lr && !(ep && i1r == i1p)) reload(i1r);
  } else {
    sweep([&](int i, float l, float E, float ld) {
      const Bounds b = bounds(i, l, E, ld);
      bool need = tiny_p ? b.live : !(b.ubp < Lp);
      if (resid) need = need || (tiny_r ? b.live : !(b.ubr < Lr)) || (!sure_any && b.live);
      if (need) reload(i);
    });
  }
  block_argmax(pv, pi, shf, shi);
  Cand c{};
  c.p_val = pv;
  c.p_idx = pi;
  if (resid) {
    block_argmax(rv, ri, shf, shi);
    any_res = __syncthreads_or(any_res);
  }
  c.r_val = rv;
  c.r_idx = ri;
  c.any_res = any_res;
  // The span's candidate out, then a count per sequence (zeroed by verify_decide): the sequence's last
  // workgroup reads every span's candidate and picks the token. No workgroup waits for another.
  __shared__ int last;
  if (threadIdx.x == 0) {
    store_cand(p.cand + (int64_t)seq * p.rchunk + chunk, c);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the candidate is stored before the count
    const int prev = __hip_atomic_fetch_add(p.done + seq, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = prev == p.rchunk - 1;
  }
  __syncthreads();
  if (last) finish_seq(p, seq, info, shf, shi);
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct VLayout {
  size_t stats, info, cand, done, total;
};

// Spans of a row: at most `most`, a multiple of 4 entries each, none empty.
void spans_of(int V, int most, int* nchunk, int* span) {
  const int n0 = std::max(1, std::min(most, (V + 3) / 4));
  *span = (((V + n0 - 1) / n0) + 3) / 4 * 4;
  *nchunk = (V + *span - 1) / *span;
}
// row_stats: at most kSpans per row (the table has S*(K+1) or more rows).
void row_spans(int V, int* nchunk, int* span) { spans_of(V, kSpans, nchunk, span); }
// verify_resample reads one target row per sequence (plus its draft row and noise): more spans per row, up
// to about 1024 workgroups in all (4 waves a SIMD, all resident at the pipelined pass's register count), so
// that a small batch still spreads over the GPU.
void resample_spans(int S, int V, int* nchunk, int* span) {
  spans_of(V, std::min(64, std::max(kSpans, (1024 + S - 1) / S)), nchunk, span);
}

VLayout verify_layout(int S, int K, int V, bool draft) {
  int nchunk, span, rchunk, rspan;
  row_spans(V, &nchunk, &span);
  resample_spans(S, V, &rchunk, &rspan);
  const int64_t rows = (int64_t)S * (K + 1) + (draft ? (int64_t)S * K : 0);
  VLayout L;
  L.stats = 0;
  L.info = align256((size_t)rows * nchunk * sizeof(RowStat));
  L.cand = align256(L.info + (size_t)S * sizeof(SeqInfo));
  L.done = align256(L.cand + (size_t)S * rchunk * sizeof(Cand));
  L.total = align256(L.done + (size_t)S * sizeof(int32_t));
  return L;
}

// Greedy-only calls (no temperatures) run the argmax pass and the decision alone; sampled calls then resample
// the sampled sequences and pick their tokens.
template <int DT, int DDT, bool kVec>
int launch_all(const VParams& p, hipStream_t s, bool draft) {
  int rc;
  if (!p.temps) {
    hipLaunchKernelGGL((row_stats<DT, DDT, kVec, false>), dim3(p.S * (p.K + 1), p.nchunk), dim3(kThreads), 0, s, p);
    if ((rc = check_launch("row_stats"))) return rc;
    hipLaunchKernelGGL((verify_decide<DT, DDT, false>), dim3(p.S), dim3(64), 0, s, p);
    return check_launch("verify_decide");
  }
  const int rows = p.S * (p.K + 1) + (draft ? p.S * p.K : 0);
  hipLaunchKernelGGL((row_stats<DT, DDT, kVec, true>), dim3(rows, p.nchunk), dim3(kThreads), 0, s, p);
  if ((rc = check_launch("row_stats"))) return rc;
  hipLaunchKernelGGL((verify_decide<DT, DDT, true>), dim3(p.S), dim3(64), 0, s, p);
  if ((rc = check_launch("verify_decide"))) return rc;
  hipLaunchKernelGGL((verify_resample<DT, DDT, kVec>), dim3(p.S, p.rchunk), dim3(kThreads), 0, s, p);
  return check_launch("verify_resample");
}

int run_verify(const char* who, const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
               const int64_t* drafts, const int64_t* num_drafts, const float* temps, const void* draft_logits,
               int32_t draft_dtype, int64_t draft_row_stride, const float* uniforms, const float* noise, int32_t S,
               int32_t K, int32_t V, int64_t* out_a, int64_t* out_next, void* workspace, size_t workspace_bytes,
               void* stream) {
  if (S < 0 || K < 0 || K > 63 || V <= 0)
    return fail(kBadArgument, "%s: bad sizes (seqs %d, draft slots %d (max 63), vocab %d)", who, S, K, V);
  if (S == 0) return kOk;
  if (!logits || !out_next || (K > 0 && (!drafts || !num_drafts)))
    return fail(kBadArgument, "%s: null pointer", who);
  if (logits_dtype != SD_DTYPE_BF16 && logits_dtype != SD_DTYPE_F32)
    return fail(kUnsupported, "%s: logits dtype %d not supported", who, logits_dtype);
  if (draft_logits && draft_dtype != SD_DTYPE_BF16 && draft_dtype != SD_DTYPE_F32)
    return fail(kUnsupported, "%s: draft dtype %d not supported", who, draft_dtype);
  if (logits_row_stride < V || (draft_logits && draft_row_stride < V))
    return fail(kBadArgument, "%s: row stride smaller than vocab", who);
  if ((int64_t)S * (K + 1) + (draft_logits ? (int64_t)S * K : 0) > 0x7fffffff || S > 0x7fffffff)
    return fail(kUnsupported, "%s: too many rows or vocabulary entries for one launch", who);
  const bool draft = draft_logits != nullptr && K > 0;
  const VLayout lay = verify_layout(S, K, V, draft);
  if (!workspace || workspace_bytes < lay.total)
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, lay.total);
  VParams p{};
  p.logits = logits;
  p.logits_stride = logits_row_stride;
  p.drafts = drafts;
  p.num_drafts = num_drafts;
  p.temps = temps;
  p.draft_logits = draft ? draft_logits : nullptr;
  p.draft_stride = draft_row_stride;
  p.uniforms = uniforms;
  p.noise = noise;
  p.S = S;
  p.K = K;
  p.V = V;
  row_spans(V, &p.nchunk, &p.span);
  resample_spans(S, V, &p.rchunk, &p.rspan);
  p.out_a = out_a;
  p.out_next = out_next;
  p.stats = (RowStat*)((uint8_t*)workspace + lay.stats);
  p.info = (SeqInfo*)((uint8_t*)workspace + lay.info);
  p.cand = (Cand*)((uint8_t*)workspace + lay.cand);
  p.done = (int32_t*)((uint8_t*)workspace + lay.done);
  hipStream_t s = (hipStream_t)stream;
  const bool lf = logits_dtype == SD_DTYPE_F32;
  const bool df = draft && draft_dtype == SD_DTYPE_F32;
  // 4-entry loads need every row (and the noise rows) aligned to 4 entries' bytes.
  auto aligned = [](const void* ptr, int64_t stride, int elem) {
    const int64_t a = 4 * elem;
    return (uintptr_t)ptr % a == 0 && (stride * elem) % a == 0;
  };
  const bool vec = aligned(logits, logits_row_stride, lf ? 4 : 2) &&
                   (!draft || aligned(draft_logits, draft_row_stride, df ? 4 : 2)) &&
                   (!noise || aligned(noise, V, 4));
  if (vec) {
    if (lf && df) return launch_all<SD_DTYPE_F32, SD_DTYPE_F32, true>(p, s, draft);
    if (lf) return launch_all<SD_DTYPE_F32, SD_DTYPE_BF16, true>(p, s, draft);
    if (df) return launch_all<SD_DTYPE_BF16, SD_DTYPE_F32, true>(p, s, draft);
    return launch_all<SD_DTYPE_BF16, SD_DTYPE_BF16, true>(p, s, draft);
  }
  if (lf && df) return launch_all<SD_DTYPE_F32, SD_DTYPE_F32, false>(p, s, draft);
  if (lf) return launch_all<SD_DTYPE_F32, SD_DTYPE_BF16, false>(p, s, draft);
  if (df) return launch_all<SD_DTYPE_BF16, SD_DTYPE_F32, false>(p, s, draft);
  return launch_all<SD_DTYPE_BF16, SD_DTYPE_BF16, false>(p, s, draft);
}

// ---- LM head + verifier ----

// The first argmax of each token row over the LM head's per-workgroup results, into the span statistics of
// a one-span row (verify_decide reads them); one wave per row, any tree order (the argmax order is total).
__global__ __launch_bounds__(64) void lm_head_merge(const lmhead::TileBest* best, int tiles, RowStat* stats) {
  const int m = blockIdx.x;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  for (int t = threadIdx.x; t < tiles; t += 64) {
    const lmhead::TileBest b = best[(int64_t)m * tiles + t];
    if (better(b.val, b.idx, bv, bi)) {
      bv = b.val;
      bi = b.idx;
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off);
    const int oi = __shfl_xor(bi, off);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (threadIdx.x == 0) stats[m] = RowStat{-INFINITY, 0.f, bv, bi};
}

// A sequence any of whose K+1 rows lists a hidden row outside [0, hidden_rows) gets num_accepted = next_token
// = -1 (the reference's logits_indices gather raises instead): a bad index never passes as a plausible token.
__global__ __launch_bounds__(64) void lm_head_poison(const int64_t* rows, int32_t hidden_rows, int32_t S, int32_t K,
                                                     int64_t* num_accepted, int64_t* next_token) {
  const int s = blockIdx.x * 64 + threadIdx.x;
  if (s >= S) return;
  bool bad = false;
  for (int j = 0; j <= K; ++j) {
    const int64_t r = rows[(int64_t)s * (K + 1) + j];
    bad |= r < 0 || r >= hidden_rows;
  }
  if (bad) {
    num_accepted[s] = -1;
    next_token[s] = -1;
  }
}

int lm_head_mb(int M) { return std::min(lmhead::kMaxMB, std::max(1, ((M + 31) / 32 + 1) / 2)); }

// Token rows of the packed hidden operand: the GEMM grid's rows of workgroups times their rows.
int64_t lm_head_mpad(int64_t M) {
  const int MB = lm_head_mb((int)std::min<int64_t>(M, 0x7fffffff));
  return (M + 64 * MB - 1) / (64 * MB) * (64 * MB);
}

// The GEMM runs one workgroup per CU. When the last round of its tiles, on a GPU of kSplitCUs CUs (MI355X's
// count), holds at most half as many tiles as there are CUs, those tiles are split along H into
// min(8, kSplitCUs / tail, H / 64) ranges (3 for the Qwen3 LM heads: 82 tiles of 594 in the last round). The choice depends on (V, H) only, never on the call's token rows
// or on the device it runs on, and every row of workgroups applies it: a token row's fp32 sums, and so its
// logits, are the same in every call (greedy speculative and plain decoding rely on it).
constexpr int kSplitCUs = 256;
struct LmSplit {
  int full, splits;
};
LmSplit lm_head_split(int V, int H) {
  const int tiles = (V + lmhead::kN - 1) / lmhead::kN;
  LmSplit r{tiles, 1};
  const int tail = tiles - (tiles - 1) / kSplitCUs * kSplitCUs;  // tiles of the last round, 1..kSplitCUs
  if (2 * tail > kSplitCUs) return r;
  const int splits = std::min({8, kSplitCUs / tail, H / (2 * lmhead::kK)});
  if (splits < 2) return r;
  r.full = tiles - tail;
  r.splits = splits;
  return r;
}

struct LmLayout {
  size_t best, stats, info, hp, part, total;
};
LmLayout lm_layout(int S, int K, int V, int H) {
  const int64_t M = (int64_t)S * (K + 1);
  const int tiles = (V + lmhead::kN - 1) / lmhead::kN;
  const LmSplit sp = lm_head_split(V, H);
  const int MB = lm_head_mb((int)M);
  const int64_t grid_rows = lm_head_mpad(M) / (64 * MB);
  const size_t part_bytes = sp.splits > 1 ? (size_t)grid_rows * (tiles - sp.full) * sp.splits * lmhead::kWaves * 2 *
                                                 MB * 16 * kWave * sizeof(float)
                                          : 0;
  LmLayout L;
  L.best = 0;
  L.stats = align256((size_t)M * tiles * sizeof(lmhead::TileBest));
  L.info = align256(L.stats + (size_t)M * sizeof(RowStat));
  L.hp = align256(L.info + (size_t)S * sizeof(SeqInfo));
  L.part = align256(L.hp + (size_t)lm_head_mpad(M) * H * 2);
  L.total = align256(L.part + part_bytes);
  return L;
}

// sd_linear past one row of 320-row workgroups, when every tile is split (fewer tiles than half the CUs: the
// model's projections), runs each tile's ranges one after another in one 128-row workgroup
// (lm_head_gemm<2, true>): the grid's rows of workgroups already fill the GPU, and the ranges' sums stay in
// registers instead of going through memory and lm_head_fixup. The sums and their order are the split's, so a
// row's outputs are the same in both forms. (With whole tiles too, as at vocabulary sizes, the 320-row
// workgroups read the weight fewer times and keep the physical split.)
constexpr int kSeqMB = 2;
bool lin_sequential(int M, int N, int K) {
  const LmSplit sp = lm_head_split(N, K);
  return M > 2 * lmhead::kMaxMB * 32 && sp.splits > 1 && sp.full == 0;
}

// Workspace of sd_linear: the packed rows, then the split tiles' fp32 sums (the physical split only).
struct LinLayout {
  size_t hp, part, total;
  int64_t mpad;  // token rows of the packed operand
};
LinLayout lin_layout(int M, int N, int K) {
  const int tiles = (N + lmhead::kN - 1) / lmhead::kN;
  const LmSplit sp = lm_head_split(N, K);
  const bool seq = lin_sequential(M, N, K);
  const int MB = lm_head_mb(M);
  LinLayout L;
  L.mpad = seq ? ((int64_t)M + 64 * kSeqMB - 1) / (64 * kSeqMB) * (64 * kSeqMB) : lm_head_mpad(M);
  const int64_t grid_rows = L.mpad / (64 * MB);
  L.hp = 0;
  L.part = align256((size_t)L.mpad * K * 2);
  L.total = align256(L.part + (sp.splits > 1 && !seq ? (size_t)grid_rows * (tiles - sp.full) * sp.splits *
                                                           lmhead::kWaves * 2 * MB * 16 * kWave * sizeof(float)
                                                     : 0));
  return L;
}

template <int MB>
int launch_lm_head_mb(const lmhead::Args& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.full + (a.tiles - a.full) * a.splits), (unsigned)(a.Mpad / (64 * MB)));
  hipLaunchKernelGGL(lmhead::lm_head_gemm<MB>, grid, dim3(lmhead::kThreads), 0, s, a);
  int rc = check_launch("lm_head_gemm");
  if (rc || a.splits == 1) return rc;
  hipLaunchKernelGGL(lmhead::lm_head_fixup<MB>, dim3((unsigned)(a.tiles - a.full), 2 * MB, grid.y), dim3(256), 0, s,
                     a);
  return check_launch("lm_head_fixup");
}

int launch_lm_head(const lmhead::Args& a, hipStream_t s) {
  switch (lm_head_mb(a.M)) {
    case 1: return launch_lm_head_mb<1>(a, s);
    case 2: return launch_lm_head_mb<2>(a, s);
    case 3: return launch_lm_head_mb<3>(a, s);
    case 4: return launch_lm_head_mb<4>(a, s);
    default: return launch_lm_head_mb<5>(a, s);
  }
}

// Scratch of the allocation-free entry point: one copy per GPU (a __device__ variable lives in every device's
// code object), held until the process ends. Its host-side name is not a device address: kernels get the
// address hipGetSymbolAddress returns on the current device, looked up once per device.
constexpr size_t kStaticScratchBytes = SD_VERIFY_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

// The scratch of the device that runs `stream`, which must be the current device (hipGetSymbolAddress answers
// for the current device only).
int static_scratch(const char* who, hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(kLaunchFailed, "%s: no current device (or device index >= %d)", who, kMaxDevices);
  hipDevice_t sdev = dev;
  if (hipStreamGetDevice(stream, &sdev) == hipSuccess && sdev != dev)
    return fail(kBadArgument, "%s: the stream belongs to device %d, the current device is %d", who, (int)sdev, dev);
  void* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!ptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ptr = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!ptr) {
      const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (err != hipSuccess || !ptr)
        return fail(kLaunchFailed, "%s: hipGetSymbolAddress(scratch) on device %d: %s", who, dev,
                    hipGetErrorString(err));
      g_scratch_ptr[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return kOk;
}

}  // namespace
}  // namespace sd

using namespace sd;

extern "C" size_t sd_verify_workspace_size(int32_t num_seqs, int32_t num_draft_slots, int32_t vocab,
                                           int32_t has_draft_logits) {
  if (num_seqs <= 0 || num_draft_slots < 0 || vocab <= 0) return 0;
  return verify_layout(num_seqs, num_draft_slots, vocab, has_draft_logits && num_draft_slots > 0).total;
}

extern "C" int sd_verify_drafts(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                                const int64_t* draft_token_ids, const int64_t* num_drafts, const float* temperatures,
                                const void* draft_logits, int32_t draft_dtype, int64_t draft_row_stride,
                                const float* uniforms, const float* exp_noise, int32_t num_seqs,
                                int32_t num_draft_slots, int32_t vocab, int64_t* num_accepted, int64_t* next_token,
                                void* workspace, size_t workspace_bytes, void* stream) {
  if (!num_accepted) return fail(kBadArgument, "sd_verify_drafts: null num_accepted");
  return run_verify("sd_verify_drafts", logits, logits_dtype, logits_row_stride, draft_token_ids, num_drafts,
                    temperatures, draft_logits, draft_dtype, draft_row_stride, uniforms, exp_noise, num_seqs,
                    num_draft_slots, vocab, num_accepted, next_token, workspace, workspace_bytes, stream);
}

extern "C" int sd_sample(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                         const float* temperatures, const float* exp_noise, int32_t num_seqs, int32_t vocab,
                         int64_t* next_token, void* workspace, size_t workspace_bytes, void* stream) {
  // K = 0: the accepted count is always 0; it goes to the tail of the workspace, never to the caller.
  const size_t need = sd_verify_workspace_size(num_seqs, 0, vocab, 0);
  if (num_seqs > 0 && (!workspace || workspace_bytes < need + (size_t)num_seqs * sizeof(int64_t)))
    return fail(kWorkspaceTooSmall, "sd_sample: workspace %zu B < %zu B", workspace_bytes,
                need + (size_t)num_seqs * sizeof(int64_t));
  int64_t* scratch_a = num_seqs > 0 ? (int64_t*)((uint8_t*)workspace + need) : nullptr;
  return run_verify("sd_sample", logits, logits_dtype, logits_row_stride, nullptr, nullptr, temperatures, nullptr,
                    SD_DTYPE_BF16, 0, nullptr, exp_noise, num_seqs, 0, vocab, scratch_a, next_token, workspace,
                    workspace_bytes, stream);
}

extern "C" int sd_verify_drafts_noalloc(const void* logits, int32_t logits_dtype, int64_t logits_row_stride,
                                        const int64_t* draft_token_ids, const int64_t* num_drafts,
                                        const float* temperatures, const void* draft_logits, int32_t draft_dtype,
                                        int64_t draft_row_stride, const float* uniforms, const float* exp_noise,
                                        int32_t num_seqs, int32_t num_draft_slots, int32_t vocab,
                                        int64_t* num_accepted, int64_t* next_token, void* stream) {
  const char* who = "sd_verify_drafts_noalloc";
  if (!num_accepted) return fail(kBadArgument, "%s: null num_accepted", who);
  if (num_seqs < 0 || num_draft_slots < 0 || num_draft_slots > 63 || vocab <= 0)
    return fail(kBadArgument, "%s: bad sizes (seqs %d, draft slots %d (max 63), vocab %d)", who, num_seqs,
                num_draft_slots, vocab);
  if (num_seqs == 0) return kOk;
  const size_t need = sd_verify_workspace_size(num_seqs, num_draft_slots, vocab, draft_logits != nullptr);
  if (need > kStaticScratchBytes)
    return fail(kUnsupported, "%s: %d sequences x %d slots need %zu B of scratch, more than the %zu B this entry "
                "point holds; use sd_verify_drafts with a workspace", who, num_seqs, num_draft_slots, need,
                kStaticScratchBytes);
  void* ws = nullptr;
  const int rc = static_scratch(who, (hipStream_t)stream, &ws);
  if (rc) return rc;
  return run_verify(who, logits, logits_dtype, logits_row_stride, draft_token_ids, num_drafts, temperatures,
                    draft_logits, draft_dtype, draft_row_stride, uniforms, exp_noise, num_seqs, num_draft_slots, vocab,
                    num_accepted, next_token, ws, kStaticScratchBytes, stream);
}

extern "C" size_t sd_lm_head_packed_weight_size(int32_t vocab, int32_t hidden_dim) {
  if (vocab <= 0 || hidden_dim <= 0 || hidden_dim % lmhead::kK) return 0;
  return (size_t)((vocab + lmhead::kN - 1) / lmhead::kN) * lmhead::kN * hidden_dim * 2;
}

extern "C" int sd_lm_head_pack_weight(const void* weight, int32_t vocab, int32_t hidden_dim, void* packed,
                                     void* stream) {
  const char* who = "sd_lm_head_pack_weight";
  if (vocab <= 0 || hidden_dim <= 0) return fail(kBadArgument, "%s: bad sizes (vocab %d, hidden %d)", who, vocab,
                                                 hidden_dim);
  if (hidden_dim % lmhead::kK)
    return fail(kUnsupported, "%s: hidden size %d is not a multiple of %d", who, hidden_dim, lmhead::kK);
  if (!weight || !packed) return fail(kBadArgument, "%s: null pointer", who);
  if (((uintptr_t)weight | (uintptr_t)packed) % 16) return fail(kUnsupported, "%s: 16-byte aligned buffers", who);
  const int tiles = (vocab + lmhead::kN - 1) / lmhead::kN;
  const int64_t chunks = (int64_t)tiles * (hidden_dim / 32) * lmhead::kN * 4;
  hipLaunchKernelGGL(lmhead::lm_head_pack_weight, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)weight, vocab, hidden_dim, tiles, (uint16_t*)packed);
  return check_launch(who);
}

extern "C" size_t sd_lm_head_verify_workspace_size(int32_t num_seqs, int32_t num_draft_slots, int32_t vocab,
                                                   int32_t hidden_dim, int32_t has_draft_logits) {
  if (num_seqs <= 0 || num_draft_slots < 0 || vocab <= 0 || hidden_dim <= 0) return 0;
  return std::max(lm_layout(num_seqs, num_draft_slots, vocab, hidden_dim).total,
                  verify_layout(num_seqs, num_draft_slots, vocab, has_draft_logits && num_draft_slots > 0).total);
}

extern "C" int sd_lm_head_verify(const void* hidden, int64_t hidden_row_stride, int32_t hidden_rows,
                                 const int64_t* logits_indices, const void* packed_weight, int32_t vocab,
                                 int32_t hidden_dim, const int64_t* draft_token_ids, const int64_t* num_drafts,
                                 const float* temperatures, const void* draft_logits, int32_t draft_dtype,
                                 int64_t draft_row_stride, const float* uniforms, const float* exp_noise, int32_t num_seqs,
                                 int32_t num_draft_slots, void* logits_out, int64_t logits_out_row_stride,
                                 int64_t* num_accepted, int64_t* next_token, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  const char* who = "sd_lm_head_verify";
  const int S = num_seqs, K = num_draft_slots, V = vocab, H = hidden_dim;
  if (S < 0 || K < 0 || K > 63 || V <= 0 || H <= 0)
    return fail(kBadArgument, "%s: bad sizes (seqs %d, draft slots %d (max 63), vocab %d, hidden %d)", who, S, K, V, H);
  if (S == 0) return kOk;
  if (H % lmhead::kK)
    return fail(kUnsupported, "%s: hidden size %d is not a multiple of %d", who, H, lmhead::kK);
  if (!hidden || !packed_weight || !num_accepted || !next_token || (K > 0 && (!draft_token_ids || !num_drafts)))
    return fail(kBadArgument, "%s: null pointer", who);
  if (hidden_row_stride < H || ((uintptr_t)hidden | (uintptr_t)packed_weight) % 16 || hidden_row_stride % 8)
    return fail(kUnsupported, "%s: hidden and weight must be 16-byte aligned rows (row stride a multiple of 8)", who);
  if (temperatures && !logits_out)
    return fail(kBadArgument, "%s: sampled rows read the logits again: logits_out is required with temperatures",
                who);
  if (logits_out && (logits_out_row_stride < V || (uintptr_t)logits_out % 2))
    return fail(kBadArgument, "%s: logits_out needs a row stride >= vocab", who);
  const int64_t M = (int64_t)S * (K + 1);
  if (M > 0x7fffffff / 64) return fail(kUnsupported, "%s: too many rows", who);
  if (hidden_rows < (logits_indices ? 1 : M))
    return fail(kBadArgument, "%s: hidden has %d rows (needs %s)", who, hidden_rows,
                logits_indices ? "at least 1" : "one per token row");
  hipStream_t s = (hipStream_t)stream;
  const LmLayout lay = lm_layout(S, K, V, H);
  const size_t need =
      std::max(lay.total, verify_layout(S, K, V, draft_logits != nullptr && K > 0).total);
  if (!workspace || workspace_bytes < need)
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, need);
  lmhead::Args a{};
  a.Mpad = (int32_t)lm_head_mpad(M);
  a.hp = (const uint16_t*)((uint8_t*)workspace + lay.hp);
  a.M = (int32_t)M;
  a.wp = (const uint16_t*)packed_weight;
  a.V = V;
  a.H = H;
  a.logits = (uint16_t*)logits_out;
  a.logits_stride = logits_out_row_stride;
  a.logits_vec = (uintptr_t)logits_out % 8 == 0 && logits_out_row_stride % 4 == 0;
  a.best = (lmhead::TileBest*)((uint8_t*)workspace + lay.best);
  a.tiles = (V + lmhead::kN - 1) / lmhead::kN;
  const LmSplit split = lm_head_split(V, H);
  a.full = split.full;
  a.splits = split.splits;
  a.part = (float*)((uint8_t*)workspace + lay.part);
  const int64_t hchunks = (int64_t)(H / 32) * a.Mpad * 4;
  hipLaunchKernelGGL(lmhead::lm_head_pack_hidden, dim3((unsigned)((hchunks + 255) / 256)), dim3(256), 0, s,
                     (const uint16_t*)hidden, hidden_row_stride, hidden_rows, logits_indices, a.M, a.Mpad, H,
                     (uint16_t*)a.hp);
  int rc = check_launch("lm_head_pack_hidden");
  if (rc) return rc;
  if ((rc = launch_lm_head(a, s))) return rc;
  auto poison = [&]() -> int {
    if (!logits_indices) return kOk;
    hipLaunchKernelGGL(lm_head_poison, dim3((unsigned)((S + 63) / 64)), dim3(64), 0, s, logits_indices, hidden_rows, S,
                       K, num_accepted, next_token);
    return check_launch("lm_head_poison");
  };
  if (temperatures) {  // sampled rows: the verifier's own passes over the stored logits
    rc = run_verify(who, logits_out, SD_DTYPE_BF16, logits_out_row_stride, draft_token_ids, num_drafts, temperatures,
                    draft_logits, draft_dtype, draft_row_stride, uniforms, exp_noise, S, K, V, num_accepted,
                    next_token, workspace, workspace_bytes, stream);
    return rc ? rc : poison();
  }
  VParams p{};
  p.logits = logits_out;  // read only for sampled rows (none here)
  p.logits_stride = logits_out_row_stride;
  p.drafts = draft_token_ids;
  p.num_drafts = num_drafts;
  p.S = S;
  p.K = K;
  p.V = V;
  p.nchunk = 1;
  p.span = V;
  p.out_a = num_accepted;
  p.out_next = next_token;
  p.stats = (RowStat*)((uint8_t*)workspace + lay.stats);
  p.info = (SeqInfo*)((uint8_t*)workspace + lay.info);
  hipLaunchKernelGGL(lm_head_merge, dim3((unsigned)M), dim3(64), 0, s, a.best, a.tiles, p.stats);
  if ((rc = check_launch("lm_head_merge"))) return rc;
  hipLaunchKernelGGL((verify_decide<SD_DTYPE_BF16, SD_DTYPE_BF16, false>), dim3(S), dim3(64), 0, s, p);
  if ((rc = check_launch("verify_decide"))) return rc;
  return poison();
}

extern "C" size_t sd_linear_workspace_size(int32_t rows, int32_t out_features, int32_t in_features) {
  if (rows <= 0 || out_features <= 0 || in_features <= 0 || in_features % lmhead::kK) return 0;
  return lin_layout(rows, out_features, in_features).total;
}

extern "C" int sd_linear(const void* x, int64_t x_row_stride, int32_t rows, const void* packed_weight,
                         int32_t out_features, int32_t in_features, void* out, int64_t out_row_stride, void* workspace,
                         size_t workspace_bytes, void* stream) {
  const char* who = "sd_linear";
  const int M = rows, N = out_features, K = in_features;
  if (M < 0 || N <= 0 || K <= 0) return fail(kBadArgument, "%s: bad sizes (rows %d, out %d, in %d)", who, M, N, K);
  if (K % lmhead::kK) return fail(kUnsupported, "%s: in_features %d is not a multiple of %d", who, K, lmhead::kK);
  if (M == 0) return kOk;
  if (M > 0x7fffffff / 64) return fail(kUnsupported, "%s: too many rows", who);
  if (!x || !packed_weight || !out) return fail(kBadArgument, "%s: null pointer", who);
  if (x_row_stride < K || out_row_stride < N)
    return fail(kBadArgument, "%s: a row stride is smaller than the row", who);
  if (((uintptr_t)x | (uintptr_t)packed_weight) % 16 || x_row_stride % 8 || (uintptr_t)out % 2)
    return fail(kUnsupported, "%s: x needs 16-byte aligned rows (row stride a multiple of 8 elements)", who);
  const LinLayout lay = lin_layout(M, N, K);
  if (!workspace || workspace_bytes < lay.total)
    return fail(kWorkspaceTooSmall, "%s: workspace %zu B < %zu B", who, workspace_bytes, lay.total);
  hipStream_t s = (hipStream_t)stream;
  lmhead::Args a{};
  a.Mpad = (int32_t)lay.mpad;
  a.hp = (const uint16_t*)((uint8_t*)workspace + lay.hp);
  a.M = M;
  a.wp = (const uint16_t*)packed_weight;
  a.V = N;
  a.H = K;
  a.logits = (uint16_t*)out;
  a.logits_stride = out_row_stride;
  a.logits_vec = (uintptr_t)out % 8 == 0 && out_row_stride % 4 == 0;
  a.best = nullptr;
  a.tiles = (N + lmhead::kN - 1) / lmhead::kN;
  const LmSplit split = lm_head_split(N, K);
  a.full = split.full;
  a.splits = split.splits;
  a.part = (float*)((uint8_t*)workspace + lay.part);
  const int64_t hchunks = (int64_t)(K / 32) * a.Mpad * 4;
  hipLaunchKernelGGL(lmhead::lm_head_pack_hidden, dim3((unsigned)((hchunks + 255) / 256)), dim3(256), 0, s,
                     (const uint16_t*)x, x_row_stride, M, (const int64_t*)nullptr, a.M, a.Mpad, K, (uint16_t*)a.hp);
  const int rc = check_launch("lm_head_pack_hidden");
  if (rc) return rc;
  if (lin_sequential(M, N, K)) {
    hipLaunchKernelGGL((lmhead::lm_head_gemm<kSeqMB, true>), dim3((unsigned)a.tiles, (unsigned)(a.Mpad / (64 * kSeqMB))),
                       dim3(lmhead::kThreads), 0, s, a);
    return check_launch("lm_head_gemm");
  }
  return launch_lm_head(a, s);
}
