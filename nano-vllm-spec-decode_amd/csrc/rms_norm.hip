// RMSNorm over hidden-state rows, with the optional residual add (nanovllm/layers/layernorm.py:16-38):
//   rms_forward      out = bf16(bf16(x * r) * w),                      r = 1 / sqrt(mean(x^2) + eps)
//   add_rms_forward  s = x + residual (fp32), residual_out = bf16(s),   out = bf16(bf16(s * r) * w), r from s
// One 256-thread workgroup per row. Thread t holds the row's 16-byte chunks t, t + 256, ...; its sum of
// squares runs over them in that order, then a fixed butterfly over the wave and the four waves' sums in wave
// order. The summation order therefore depends on the hidden size alone: a row's result is bitwise the same
// whatever the number of rows in the call, which keeps a model's greedy tokens independent of the batch (the
// library reductions split a short batch's rows across more threads). The arithmetic after the sum follows
// the reference's eager operations (fp32 mean, correctly rounded square root and reciprocal, two roundings
// to bf16), so its only difference from them is the order of the sum of squares.
#include <algorithm>

#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunks = 8;  // 16-byte chunks per thread: rows of up to 16384 elements

struct NormArgs {
  const uint16_t* x;
  const uint16_t* residual;  // null: rms_forward
  const uint16_t* weight;
  uint16_t* out;
  uint16_t* residual_out;    // with residual
  int64_t x_stride, residual_stride, out_stride, residual_out_stride;
  int32_t hidden;
  float eps;
};

__device__ __forceinline__ void unpack8(const uint4& u, float* f) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __builtin_bit_cast(float, w[i] << 16);
    f[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint4 pack8(const float* f) {
  return make_uint4(cvt_bf16x2(f[0], f[1]), cvt_bf16x2(f[2], f[3]), cvt_bf16x2(f[4], f[5]),
                    cvt_bf16x2(f[6], f[7]));
}

__device__ __forceinline__ float to_bf16(float f) { return __builtin_bit_cast(float, cvt_bf16x2(f, 0.0f) << 16); }

template <int NC>
__global__ __launch_bounds__(kThreads) void rms_norm_rows(NormArgs a) {
#pragma clang fp contract(off)
  __shared__ float wave_sums[kThreads / kWave];
  const int64_t row = blockIdx.x;
  const int t = threadIdx.x;
  const int chunks = a.hidden / 8;
  const uint16_t* x = a.x + row * a.x_stride;
  float v[NC][8];
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = t + i * kThreads;
    if (c < chunks) {
      unpack8(*(const uint4*)(x + 8 * c), v[i]);
      if (a.residual) {
        float r[8];
        unpack8(*(const uint4*)(a.residual + row * a.residual_stride + 8 * c), r);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[i][e] += r[e];
        *(uint4*)(a.residual_out + row * a.residual_out_stride + 8 * c) = pack8(v[i]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[i][e] * v[i][e];
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
  if (t % kWave == 0) wave_sums[t / kWave] = ss;
  __syncthreads();
  float total = wave_sums[0];
#pragma unroll
  for (int w = 1; w < kThreads / kWave; ++w) total += wave_sums[w];
  // torch.rsqrt(var + eps) as 1 / sqrt, both correctly rounded: the root in fp64 rounded to fp32 is the
  // correctly rounded fp32 root (an exact root of an fp32 value never lies within 2^-52 of an fp32 midpoint).
  const float var = __fdiv_rn(total, (float)a.hidden);
  const float r = __fdiv_rn(1.0f, (float)__dsqrt_rn((double)(var + a.eps)));
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int c = t + i * kThreads;
    if (c < chunks) {
      float w[8];
      unpack8(*(const uint4*)(a.weight + 8 * c), w);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[i][e] = to_bf16(to_bf16(v[i][e] * r) * w[e]);
      *(uint4*)(a.out + row * a.out_stride + 8 * c) = pack8(v[i]);
    }
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace sd

using namespace sd;

extern "C" int sd_rms_norm(const void* x, int64_t x_row_stride, const void* residual, int64_t residual_row_stride,
                           const void* weight, float eps, int32_t rows, int32_t hidden, void* out,
                           int64_t out_row_stride, void* residual_out, int64_t residual_out_row_stride, void* stream) {
  const char* who = "sd_rms_norm";
  if (rows < 0 || hidden <= 0) return fail(kBadArgument, "%s: bad sizes (rows %d, hidden %d)", who, rows, hidden);
  if (hidden % 8 || hidden > 8 * kThreads * kMaxChunks)
    return fail(kUnsupported, "%s: hidden size %d (a multiple of 8, at most %d)", who, hidden,
                8 * kThreads * kMaxChunks);
  if (!(eps >= 0.0f) || eps == __builtin_inff()) return fail(kBadArgument, "%s: eps must be finite and >= 0", who);
  if ((residual == nullptr) != (residual_out == nullptr))
    return fail(kBadArgument, "%s: give residual and residual_out together", who);
  if (rows == 0) return kOk;
  if (!x || !weight || !out) return fail(kBadArgument, "%s: null pointer", who);
  if (x_row_stride < hidden || out_row_stride < hidden ||
      (residual && (residual_row_stride < hidden || residual_out_row_stride < hidden)))
    return fail(kBadArgument, "%s: a row stride is smaller than the hidden size", who);
  const bool ok = aligned16(x) && aligned16(weight) && aligned16(out) && x_row_stride % 8 == 0 &&
                  out_row_stride % 8 == 0 &&
                  (!residual || (aligned16(residual) && aligned16(residual_out) && residual_row_stride % 8 == 0 &&
                                 residual_out_row_stride % 8 == 0));
  if (!ok) return fail(kUnsupported, "%s: pointers must be 16-byte aligned and row strides multiples of 8", who);
  NormArgs a;
  a.x = (const uint16_t*)x;
  a.residual = (const uint16_t*)residual;
  a.weight = (const uint16_t*)weight;
  a.out = (uint16_t*)out;
  a.residual_out = (uint16_t*)residual_out;
  a.x_stride = x_row_stride;
  a.residual_stride = residual_row_stride;
  a.out_stride = out_row_stride;
  a.residual_out_stride = residual_out_row_stride;
  a.hidden = hidden;
  a.eps = eps;
  const int nc = (hidden / 8 + kThreads - 1) / kThreads;
  const dim3 grid((uint32_t)rows), block(kThreads);
  hipStream_t s = (hipStream_t)stream;
  switch (nc) {
    case 1: hipLaunchKernelGGL(rms_norm_rows<1>, grid, block, 0, s, a); break;
    case 2: hipLaunchKernelGGL(rms_norm_rows<2>, grid, block, 0, s, a); break;
    case 3:
    case 4: hipLaunchKernelGGL(rms_norm_rows<4>, grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL(rms_norm_rows<kMaxChunks>, grid, block, 0, s, a); break;
  }
  return check_launch(who);
}
