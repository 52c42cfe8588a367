// Fused q/k RMSNorm + rotary embedding + paged KV store: the per-token work between the qkv projection
// and attention (nanovllm/models/qwen3.py:83-97, then the store of nanovllm/layers/attention.py:33-40).
//
// One 8-lane group per (token, head) of the qkv row; a token's heads fill one workgroup (blockIdx.x = token,
// 48 heads x 8 lanes = 384 threads for Qwen3-8B), in row order (q heads, then k, then v), so consecutive
// groups read consecutive 256-byte head rows and the token's position and slot are scalar loads. Lane c
// holds elements 8c..8c+7 of each half of the head (the halves the neox rotation pairs): two 16-byte loads.
//   q / k heads: fp32 sum of squares over the head (8-lane butterfly), x * (1 / sqrt(mean + eps)) rounded
//                to bf16, times the bf16 weight rounded to bf16 (skipped for models without q/k norm),
//                then the rotation by the fp32 cos / sin row of the token's position, rounded to bf16.
//                q goes to q_out; k goes to k_out (optional) and to the token's k-cache slot.
//   v heads:     copied to the token's v-cache slot (only launched when the caches are given).
// The arithmetic follows the reference's eager operations one by one (correctly rounded sqrt and divide,
// no fused multiply-adds), so its only difference from them is the order of the 128-term sum of squares.
// A position outside [0, max_position) uses NaN for cos and sin: that token's q / k come out NaN instead
// of reading outside the table.
#include <algorithm>

#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {
namespace {

constexpr int kHeadDim = 128;
constexpr int kHalf = kHeadDim / 2;
constexpr int kLanesPerHead = 8;  // 8 lanes x (8 + 8) elements = one head

struct NormRopeArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_stride, k_stride, v_stride;
  const int64_t* positions;
  const uint16_t* q_weight;  // null: no norm (then k_weight is null too)
  const uint16_t* k_weight;
  const float* cos_sin;  // [max_position, kHeadDim]: cos of the kHalf frequencies, then sin
  int64_t max_position;
  uint16_t* q_out;
  uint16_t* k_out;  // null: k only goes to the cache
  int64_t q_out_stride, k_out_stride;
  uint16_t* k_cache;  // null: no store (then no v groups are launched)
  uint16_t* v_cache;
  int64_t num_slots;
  const int32_t* slots;
  float eps;
  int32_t num_tokens, Hq, Hkv, Hv;  // Hv = Hkv with caches, else 0
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

// The fp32 value of f rounded to bf16 (round to nearest even).
__device__ __forceinline__ float to_bf16(float f) {
  return __builtin_bit_cast(float, cvt_bf16x2(f, 0.0f) << 16);
}

// y = (x rounded after * r) * w rounded: RMSNorm's two roundings (layernorm.py:23-25), in place.
__device__ __forceinline__ void scale_weight(float* x, float r, const uint4& wu) {
  float w[8];
  unpack8(wu, w);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = to_bf16(to_bf16(x[i] * r) * w[i]);
}

__global__ __launch_bounds__(1024) void qk_norm_rope_store(NormRopeArgs a) {
#pragma clang fp contract(off)
  const int Htot = a.Hq + a.Hkv + a.Hv;
  // One token per workgroup row (blockIdx.x): its position and slot are workgroup-uniform (scalar loads,
  // issued first so that the cos / sin row address is known early).
  const int64_t t = blockIdx.x;
  const int64_t pos = a.positions[t];
  const int64_t slot_raw = a.k_cache != nullptr ? (int64_t)a.slots[t] : -1;
  const int h = (int)((blockIdx.y * blockDim.x + threadIdx.x) / kLanesPerHead);
  const int c = threadIdx.x % kLanesPerHead;
  if (h >= Htot) return;
  const int kind = h < a.Hq ? 0 : (h < a.Hq + a.Hkv ? 1 : 2);  // q, k, v
  const int hh = kind == 0 ? h : (kind == 1 ? h - a.Hq : h - a.Hq - a.Hkv);
  const uint16_t* src = (kind == 0 ? a.q + t * a.q_stride : kind == 1 ? a.k + t * a.k_stride : a.v + t * a.v_stride) +
                        (int64_t)hh * kHeadDim + c * 8;
  const uint4 u1 = *(const uint4*)src;
  const uint4 u2 = *(const uint4*)(src + kHalf);
  int64_t slot = -1;
  if (kind != 0) {
    slot = slot_raw;
    if (slot >= a.num_slots) slot = -1;
  }
  const int64_t cache_off = slot * ((int64_t)a.Hkv * kHeadDim) + (int64_t)hh * kHeadDim + c * 8;
  if (kind == 2) {
    if (slot >= 0) {
      *(uint4*)(a.v_cache + cache_off) = u1;
      *(uint4*)(a.v_cache + cache_off + kHalf) = u2;
    }
    return;
  }
  const bool pos_ok = pos >= 0 && pos < a.max_position;
  const float* cs = a.cos_sin + (pos_ok ? pos : 0) * kHeadDim + c * 8;
  const float4 c0 = *(const float4*)cs, c1 = *(const float4*)(cs + 4);
  const float4 s0 = *(const float4*)(cs + kHalf), s1 = *(const float4*)(cs + kHalf + 4);
  const uint16_t* w = kind == 0 ? a.q_weight : a.k_weight;
  uint4 w1 = make_uint4(0, 0, 0, 0), w2 = w1;
  if (w != nullptr) {
    w1 = *(const uint4*)(w + c * 8);
    w2 = *(const uint4*)(w + kHalf + c * 8);
  }

  float x1[8], x2[8];
  unpack8(u1, x1);
  unpack8(u2, x2);
  if (w != nullptr) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += x1[i] * x1[i];
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += x2[i] * x2[i];
    ss += __shfl_xor(ss, 1, kLanesPerHead);
    ss += __shfl_xor(ss, 2, kLanesPerHead);
    ss += __shfl_xor(ss, 4, kLanesPerHead);
    // torch.rsqrt on fp32 is 1 / sqrt with both steps correctly rounded. v_sqrt_f32 is not (1 ulp), so the
    // root is taken in fp64 (correctly rounded) and rounded to fp32: the exact root of an fp32 value is never
    // within 2^-52 (relative) of an fp32 rounding midpoint, so this second rounding is exact too.
    const float root = (float)__dsqrt_rn((double)(ss * (1.0f / kHeadDim) + a.eps));
    const float r = __fdiv_rn(1.0f, root);
    scale_weight(x1, r, w1);
    scale_weight(x2, r, w2);
  }

  const float nan = __builtin_nanf("");
  const float cosv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sinv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  float y1[8], y2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float co = pos_ok ? cosv[i] : nan, si = pos_ok ? sinv[i] : nan;
    y1[i] = x1[i] * co - x2[i] * si;
    y2[i] = x2[i] * co + x1[i] * si;
  }
  const uint4 o1 = pack8(y1), o2 = pack8(y2);
  uint16_t* dst = kind == 0 ? a.q_out + t * a.q_out_stride : (a.k_out ? a.k_out + t * a.k_out_stride : nullptr);
  if (dst != nullptr) {
    dst += (int64_t)hh * kHeadDim + c * 8;
    *(uint4*)dst = o1;
    *(uint4*)(dst + kHalf) = o2;
  }
  if (slot >= 0) {
    *(uint4*)(a.k_cache + cache_off) = o1;
    *(uint4*)(a.k_cache + cache_off + kHalf) = o2;
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace sd

using namespace sd;

extern "C" int sd_qk_norm_rope_store(const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride,
                                     const void* v, int64_t v_row_stride, const int64_t* positions,
                                     const void* q_norm_weight, const void* k_norm_weight, float eps,
                                     const float* cos_sin_cache, int64_t max_position, void* q_out,
                                     int64_t q_out_row_stride, void* k_out, int64_t k_out_row_stride,
                                     void* k_cache, void* v_cache, int64_t num_slots,
                                     const int32_t* slot_mapping, int32_t num_tokens, int32_t num_heads,
                                     int32_t num_kv_heads, int32_t head_dim, void* stream) {
  const char* who = "sd_qk_norm_rope_store";
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || max_position <= 0)
    return fail(kBadArgument, "%s: bad sizes (tokens %d, heads %d, kv heads %d, head_dim %d, max_position %lld)",
                who, num_tokens, num_heads, num_kv_heads, head_dim, (long long)max_position);
  if (head_dim != kHeadDim) return fail(kUnsupported, "%s: head_dim %d (only %d)", who, head_dim, kHeadDim);
  if (!(eps >= 0.0f) || eps == __builtin_inff()) return fail(kBadArgument, "%s: eps must be finite and >= 0", who);
  if ((q_norm_weight == nullptr) != (k_norm_weight == nullptr))
    return fail(kBadArgument, "%s: give both norm weights or neither", who);
  const bool store = k_cache != nullptr || v_cache != nullptr;
  if (store && (k_cache == nullptr || v_cache == nullptr || v == nullptr || slot_mapping == nullptr || num_slots < 0))
    return fail(kBadArgument, "%s: the store needs k_cache, v_cache, v, slot_mapping and num_slots >= 0", who);
  if (num_tokens == 0) return kOk;
  if (!q || !k || !positions || !cos_sin_cache || !q_out) return fail(kBadArgument, "%s: null pointer", who);
  const int64_t qw = (int64_t)num_heads * head_dim, kw = (int64_t)num_kv_heads * head_dim;
  if (q_row_stride < qw || q_out_row_stride < qw || k_row_stride < kw || (k_out && k_out_row_stride < kw) ||
      (store && v_row_stride < kw))
    return fail(kBadArgument, "%s: a row stride is smaller than heads * head_dim", who);
  const bool strides8 = q_row_stride % 8 == 0 && k_row_stride % 8 == 0 && q_out_row_stride % 8 == 0 &&
                        (!k_out || k_out_row_stride % 8 == 0) && (!store || v_row_stride % 8 == 0);
  const bool ptrs16 = aligned16(q) && aligned16(k) && aligned16(q_out) && aligned16(cos_sin_cache) &&
                      (!k_out || aligned16(k_out)) && (!store || (aligned16(v) && aligned16(k_cache) && aligned16(v_cache))) &&
                      (!q_norm_weight || (aligned16(q_norm_weight) && aligned16(k_norm_weight)));
  if (!strides8 || !ptrs16)
    return fail(kUnsupported, "%s: pointers must be 16-byte aligned and row strides multiples of 8 elements", who);

  NormRopeArgs a;
  a.q = (const uint16_t*)q;
  a.k = (const uint16_t*)k;
  a.v = (const uint16_t*)v;
  a.q_stride = q_row_stride;
  a.k_stride = k_row_stride;
  a.v_stride = v_row_stride;
  a.positions = positions;
  a.q_weight = (const uint16_t*)q_norm_weight;
  a.k_weight = (const uint16_t*)k_norm_weight;
  a.cos_sin = cos_sin_cache;
  a.max_position = max_position;
  a.q_out = (uint16_t*)q_out;
  a.k_out = (uint16_t*)k_out;
  a.q_out_stride = q_out_row_stride;
  a.k_out_stride = k_out_row_stride;
  a.k_cache = (uint16_t*)k_cache;
  a.v_cache = (uint16_t*)v_cache;
  a.num_slots = num_slots;
  a.slots = slot_mapping;
  a.eps = eps;
  a.num_tokens = num_tokens;
  a.Hq = num_heads;
  a.Hkv = num_kv_heads;
  a.Hv = store ? num_kv_heads : 0;
  // A token's heads in one workgroup row: 8 lanes a head, up to 1024 threads a workgroup.
  const int lanes = (num_heads + num_kv_heads + a.Hv) * kLanesPerHead;
  const int threads = std::min(1024, (lanes + 63) / 64 * 64);
  const int rows = (lanes + threads - 1) / threads;
  if (rows > 65535) return fail(kUnsupported, "%s: too many heads (%d)", who, num_heads + num_kv_heads);
  hipLaunchKernelGGL(qk_norm_rope_store, dim3((uint32_t)num_tokens, (uint32_t)rows), dim3(threads), 0,
                     (hipStream_t)stream, a);
  return check_launch(who);
}
