// Speculative-decoding verifier and token sampler over the full vocabulary (replaces verify_drafts and
// Sampler.forward, nanovllm/layers/sampler.py:5-103).
//
// Four kernels, two of them HBM-streaming over [rows, vocab] tables. A row is cut into at most
// kSpans contiguous spans (a multiple of 4 entries each, none empty); a 256-thread workgroup streams one
// span with 4-entry loads (16 B for fp32, 8 B for bf16; scalar loads when the rows are not aligned).
//   1. row_stats      (row, span): first argmax of the raw logits of target rows; for rows with temperature
//                     != 0 also max and sum(exp(x - max)) of x = l / T (target rows and, when given, draft
//                     rows), kept per thread online and combined in a fixed order.
//   2. verify_decide  (seq): merges span stats in span order (argmax, logsumexp), applies the accept rule
//                     u * q(d) < p(d) (or top1 == d for greedy rows) to the leading run of real guesses,
//                     writes num_accepted and, for greedy rows, next_token.
//   3. verify_resample(seq, span): random rows only, over up to 64 spans per row (a single row per
//                     sequence: more spans keep a small batch spread over the GPU): the first argmax of
//                     p / max(E, 1e-10) and of
//                     residual / max(E, 1e-10) with p = softmax(row a / T), residual = max(p - q, 0) (or p
//                     with the rejected n-gram guess zeroed), and whether any residual is positive.
//   4. verify_finish  (seq): random rows only: merges the span candidates and picks the token.
// Every reduction has a fixed order, so results are deterministic; ties resolve to the first index (and a
// NaN counts as the largest value), as torch.argmax does.
#include <math.h>

#include <algorithm>
#include <atomic>
#include <mutex>

#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {
namespace {

constexpr int kSpans = 8;         // most spans per row (workgroups per row)
constexpr int kThreads = 256;

struct RowStat {                  // per (row, chunk)
  float max_x;                    // max of l / T over the chunk (random rows; -inf for an all -inf chunk)
  float sum;                      // sum of exp(l / T - lse_shift(max_x)) (random rows)
  float best;                     // raw logit at the chunk's first argmax (target rows)
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

// true if (v, i) should replace (bv, bi) under torch.argmax order: NaN largest, then value, then lower index.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

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

// The shift of a logsumexp: the maximum, or 0 when it is infinite (torch.logsumexp's rule), so that
// an all -inf set sums to 0 (lse -inf) and a +inf entry gives +inf.
__device__ __forceinline__ float lse_shift(float m) { return fabsf(m) == INFINITY ? 0.f : m; }

// Online (max m, sum s of exp(x - lse_shift(m))) of one thread's entries. s == 0 exactly while every entry
// seen is -inf; a rescale is skipped then (it would multiply 0 by an overflowing factor).
struct OnlineSum {
  float m = -INFINITY, s = 0.f;
  __device__ __forceinline__ void add4(float x0, float x1, float x2, float x3) {
    const float ml = fmaxf(fmaxf(x0, x1), fmaxf(x2, x3));
    if (ml > m) {
      if (s != 0.f) s *= exp_acc(lse_shift(m) - lse_shift(ml));
      m = ml;
    }
    const float sh = lse_shift(m);
    s += exp_acc(x0 - sh) + exp_acc(x1 - sh) + exp_acc(x2 - sh) + exp_acc(x3 - sh);
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
};

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
  const void* base;
  if (is_target) {
    base = DT == SD_DTYPE_F32 ? (const void*)((const float*)p.logits + (int64_t)row * p.logits_stride)
                              : (const void*)((const uint16_t*)p.logits + (int64_t)row * p.logits_stride);
  } else {
    const int64_t dr = row - target_rows;
    base = DDT == SD_DTYPE_F32 ? (const void*)((const float*)p.draft_logits + dr * p.draft_stride)
                               : (const void*)((const uint16_t*)p.draft_logits + dr * p.draft_stride);
  }
  const int v0 = chunk * p.span;
  const int v1 = min(v0 + p.span, p.V);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  OnlineSum os;
  auto visit = [&](float raw, int v) {  // scalar entry
    if (is_target && better(raw, v, bv, bi)) {
      bv = raw;
      bi = v;
    }
  };
  auto load4 = [&](int v) {
    return is_target ? load_logit4<DT>(base, v) : load_logit4<DDT>(base, v);
  };
  auto body = [&](int v, const float (&r)[4]) {  // entries v .. v+3 (those below v1)
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (v + e < v1) visit(r[e], v + e);
    if (random) {
      float x[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = v + e < v1 ? (T == 1.f ? r[e] : r[e] / T) : -INFINITY;  // x / 1 == x
      os.add4(x[0], x[1], x[2], x[3]);
    }
  };
  // A thread visits v0 + 4*tid, then every 4*kThreads entries, in increasing order; the aligned main loop
  // issues four of those loads before using any (the same visiting order, more loads in flight).
  constexpr int kStep = 4 * kThreads;
  int v = v0 + 4 * threadIdx.x;
  if (kVec) {
    for (; v + 3 * kStep + 4 <= v1; v += 4 * kStep) {
      float4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = load4(v + u * kStep);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float r[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
        body(v + u * kStep, r);
      }
    }
  }
  for (; v < v1; v += kStep) {
    float r[4];
    if (kVec && v + 4 <= v1) {
      const float4 q4 = load4(v);
      r[0] = q4.x;
      r[1] = q4.y;
      r[2] = q4.z;
      r[3] = q4.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        r[e] = v + e < v1 ? (is_target ? load_logit<DT>(base, v + e) : load_logit<DDT>(base, v + e)) : -INFINITY;
    }
    body(v, r);
  }
  RowStat st;
  st.max_x = -INFINITY;
  st.sum = 0.f;
  if (is_target) block_argmax(bv, bi, shf, shi);
  st.best = bv;
  st.best_idx = bi;
  if (random) {
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

template <int DT, int DDT, bool kRand>
__global__ __launch_bounds__(64) void verify_decide(VParams p) {
  __shared__ int32_t top1[65];
  __shared__ float lse[65];
  __shared__ float dlse[64];
  const int seq = blockIdx.x;
  const int lane = threadIdx.x;
  const int K = p.K;
  const float T = kRand ? p.temps[seq] : 0.f;
  const bool random = kRand && T != 0.f;
  const int target_rows = p.S * (K + 1);
  for (int j = lane; j <= K; j += 64) {
    const RowStat* st = p.stats + (int64_t)(seq * (K + 1) + j) * p.nchunk;
    float bv = st[0].best;
    int bi = st[0].best_idx;
    for (int c = 1; c < p.nchunk; ++c)
      if (better(st[c].best, st[c].best_idx, bv, bi)) {
        bv = st[c].best;
        bi = st[c].best_idx;
      }
    top1[j] = bi;
    if (random) {
      float M, s;
      merge_softmax(st, p.nchunk, &M, &s);
      lse[j] = logf(s) + M;
    }
  }
  if (random && p.draft_logits) {
    for (int j = lane; j < K; j += 64) {
      const RowStat* st = p.stats + (int64_t)(target_rows + seq * K + j) * p.nchunk;
      float M, s;
      merge_softmax(st, p.nchunk, &M, &s);
      dlse[j] = logf(s) + M;
    }
  }
  __syncthreads();
  // Each lane evaluates one guess (the scattered loads run in parallel), lane 0 takes the leading run.
  __shared__ int accj[64];
  const int64_t nd = p.num_drafts ? p.num_drafts[seq] : 0;
  for (int j = lane; j < K; j += 64) {
    const int64_t d = p.drafts[(int64_t)seq * K + j];
    bool acc = false;
    if (j < nd && d >= 0 && d < p.V) {
      if (!random) {
        acc = top1[j] == d;
      } else {
        const float xl = (DT == SD_DTYPE_F32)
                             ? ((const float*)p.logits)[(int64_t)(seq * (K + 1) + j) * p.logits_stride + d]
                             : bf16_bits_to_f32(((const uint16_t*)p.logits)[(int64_t)(seq * (K + 1) + j) * p.logits_stride + d]);
        const float pd = exp_acc(xl / T - lse[j]);
        float qd = 1.f;
        if (p.draft_logits) {
          const int64_t dr = (int64_t)seq * K + j;
          const float xd = (DDT == SD_DTYPE_F32)
                               ? ((const float*)p.draft_logits)[dr * p.draft_stride + d]
                               : bf16_bits_to_f32(((const uint16_t*)p.draft_logits)[dr * p.draft_stride + d]);
          qd = exp_acc(xd / T - dlse[j]);
        }
        const float u = p.uniforms ? p.uniforms[(int64_t)seq * K + j] : 1.f;  // missing uniforms: u = 1
        acc = u * qd < pd;
      }
    }
    accj[j] = acc ? 1 : 0;
  }
  __syncthreads();
  if (lane != 0) return;
  int a = 0;
  while (a < K && accj[a]) ++a;
  p.out_a[seq] = a;
  SeqInfo info{};
  info.a = a;
  info.random = random ? 1 : 0;
  info.guess = -1;
  if (!random) {
    p.out_next[seq] = top1[a];
  } else {
    const RowStat* st = p.stats + (int64_t)(seq * (K + 1) + a) * p.nchunk;
    merge_softmax(st, p.nchunk, &info.Ma, &info.Sa);
    info.rejected = a < nd ? 1 : 0;
    if (K > 0) {
      const int j = min(a, K - 1);
      const int64_t d = p.drafts[(int64_t)seq * K + j];
      if (p.draft_logits) {
        info.resid_mode = 2;
        merge_softmax(p.stats + (int64_t)(target_rows + seq * K + j) * p.nchunk, p.nchunk, &info.Md, &info.Sd);
      } else {
        info.resid_mode = 1;
        info.guess = (d >= 0 && d < p.V) ? (int32_t)d : -1;
      }
    }
  }
  p.info[seq] = info;
}

// One workgroup per random sequence: thread k reads span k's candidate (all reads in flight together),
// then the same block reductions as inside a span. The argmax order (value, then lower index) makes the
// result independent of the reduction tree. A kernel of its own: merging in the last span workgroup would
// need device-scope fences (an L2 write-back and invalidate per workgroup on this GPU), which cost more
// than the launch.
__global__ __launch_bounds__(kThreads) void verify_finish(VParams p) {
  __shared__ float shf[4];
  __shared__ int shi[4];
  const int seq = blockIdx.x;
  const SeqInfo info = p.info[seq];
  if (!info.random) return;
  float pv = -INFINITY, rv = -INFINITY;
  int pi = 0x7fffffff, ri = 0x7fffffff, any_res = 0;
  for (int k = threadIdx.x; k < p.rchunk; k += kThreads) {
    const Cand c = p.cand[(int64_t)seq * p.rchunk + k];
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

template <int DT, int DDT, bool kVec>
__global__ __launch_bounds__(kThreads) void verify_resample(VParams p) {
  __shared__ float shf[4];
  __shared__ int shi[4];
  const int seq = blockIdx.x;
  const int chunk = blockIdx.y;
  const SeqInfo info = p.info[seq];
  if (!info.random) return;
  const float T = p.temps[seq];
  const int K = p.K;
  const int64_t trow = (int64_t)seq * (K + 1) + info.a;
  const int64_t drow = (int64_t)seq * K + min(info.a, K - 1);
  const void* tbase = DT == SD_DTYPE_F32 ? (const void*)((const float*)p.logits + trow * p.logits_stride)
                                         : (const void*)((const uint16_t*)p.logits + trow * p.logits_stride);
  const void* dbase = nullptr;
  if (info.resid_mode == 2)
    dbase = DDT == SD_DTYPE_F32 ? (const void*)((const float*)p.draft_logits + drow * p.draft_stride)
                                : (const void*)((const uint16_t*)p.draft_logits + drow * p.draft_stride);
  const float* noise = p.noise ? p.noise + (int64_t)seq * p.V : nullptr;  // missing noise: E = 1
  const int v0 = chunk * p.rspan;
  const int v1 = min(v0 + p.rspan, p.V);
  float pv = -INFINITY, rv = -INFINITY;
  int pi = 0x7fffffff, ri = 0x7fffffff;
  int any_res = 0;
  auto body = [&](int v, const float (&l)[4], const float (&E)[4], const float (&ld)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = v + e;
      if (idx >= v1) continue;
      float prob = exp_acc((T == 1.f ? l[e] : l[e] / T) - info.Ma) / info.Sa;
      const float Ee = noise ? fmaxf(E[e], 1e-10f) : 1.f;
      if (info.resid_mode == 1 && info.rejected && idx == info.guess) prob = 0.f;
      const float sp = prob / Ee;
      if (better(sp, idx, pv, pi)) {
        pv = sp;
        pi = idx;
      }
      if (dbase) {
        const float q = exp_acc((T == 1.f ? ld[e] : ld[e] / T) - info.Md) / info.Sd;
        const float res = fmaxf(prob - q, 0.f);
        any_res |= res > 0.f;
        const float sr = res / Ee;
        if (better(sr, idx, rv, ri)) {
          rv = sr;
          ri = idx;
        }
      }
    }
  };
  // Same per-thread visiting order as row_stats; the aligned main loop has the loads of two steps (target,
  // noise and draft rows) in flight before using them.
  constexpr int kStep = 4 * kThreads;
  int v = v0 + 4 * threadIdx.x;
  if (kVec) {
    for (; v + kStep + 4 <= v1; v += 2 * kStep) {
      float4 t4[2], e4[2], d4[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        t4[u] = load_logit4<DT>(tbase, v + u * kStep);
        e4[u] = noise ? *(const float4*)(noise + v + u * kStep) : make_float4(1.f, 1.f, 1.f, 1.f);
        d4[u] = dbase ? load_logit4<DDT>(dbase, v + u * kStep) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const float l[4] = {t4[u].x, t4[u].y, t4[u].z, t4[u].w};
        const float E[4] = {e4[u].x, e4[u].y, e4[u].z, e4[u].w};
        const float ld[4] = {d4[u].x, d4[u].y, d4[u].z, d4[u].w};
        body(v + u * kStep, l, E, ld);
      }
    }
  }
  for (; v < v1; v += kStep) {
    float l[4], E[4] = {1.f, 1.f, 1.f, 1.f}, ld[4] = {0.f, 0.f, 0.f, 0.f};
    if (kVec && v + 4 <= v1) {
      const float4 t4 = load_logit4<DT>(tbase, v);
      l[0] = t4.x, l[1] = t4.y, l[2] = t4.z, l[3] = t4.w;
      if (noise) {
        const float4 e4 = *(const float4*)(noise + v);
        E[0] = e4.x, E[1] = e4.y, E[2] = e4.z, E[3] = e4.w;
      }
      if (dbase) {
        const float4 d4 = load_logit4<DDT>(dbase, v);
        ld[0] = d4.x, ld[1] = d4.y, ld[2] = d4.z, ld[3] = d4.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const bool in = v + e < v1;
        l[e] = in ? load_logit<DT>(tbase, v + e) : 0.f;
        if (noise) E[e] = in ? noise[v + e] : 1.f;
        if (dbase) ld[e] = in ? load_logit<DDT>(dbase, v + e) : 0.f;
      }
    }
    body(v, l, E, ld);
  }
  block_argmax(pv, pi, shf, shi);
  Cand c{};
  c.p_val = pv;
  c.p_idx = pi;
  if (info.resid_mode == 2) {
    block_argmax(rv, ri, shf, shi);
    any_res = __syncthreads_or(any_res);
  }
  c.r_val = rv;
  c.r_idx = ri;
  c.any_res = any_res;
  if (threadIdx.x == 0) p.cand[(int64_t)seq * p.rchunk + chunk] = c;
}

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct VLayout {
  size_t stats, info, cand, total;
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
// to about 2048 workgroups in all, so that a small batch still spreads over the GPU.
void resample_spans(int S, int V, int* nchunk, int* span) {
  spans_of(V, std::min(64, std::max(kSpans, (2048 + S - 1) / S)), nchunk, span);
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
  L.total = align256(L.cand + (size_t)S * rchunk * sizeof(Cand));
  return L;
}

// Greedy-only calls (no temperatures) run the argmax pass and the decision alone.
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
  if ((rc = check_launch("verify_resample"))) return rc;
  hipLaunchKernelGGL(verify_finish, dim3(p.S), dim3(kThreads), 0, s, p);
  return check_launch("verify_finish");
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

// Scratch of the allocation-free entry point: one copy per GPU (a __device__ variable lives in every device's
// code object), held until the process ends. Its host-side name is not a device address: kernels get the
// address hipGetSymbolAddress returns on the current device, looked up once per device.
constexpr size_t kStaticScratchBytes = SD_VERIFY_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];
std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

int static_scratch(const char* who, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(kLaunchFailed, "%s: no current device (or device index >= %d)", who, kMaxDevices);
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
  const int rc = static_scratch(who, &ws);
  if (rc) return rc;
  return run_verify(who, logits, logits_dtype, logits_row_stride, draft_token_ids, num_drafts, temperatures,
                    draft_logits, draft_dtype, draft_row_stride, uniforms, exp_noise, num_seqs, num_draft_slots, vocab,
                    num_accepted, next_token, ws, kStaticScratchBytes, stream);
}
