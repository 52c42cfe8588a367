// Paged KV-cache scatter (replaces the Triton store_kvcache_kernel, nanovllm/layers/attention.py:10-40).
//
// One wave64 per token row. A row is num_kv_heads*head_dim bf16 elements (2 KiB for Qwen3-8B), copied
// with 16-byte vector loads/stores: each lane moves 2 x 16 B of K and 2 x 16 B of V, all loads issued
// before the stores (the first ones together with the slot's load). A negative slot (-1 = graph padding)
// stores nothing.
#include "sd_common.h"
#include "../../include/sd_attn.h"

namespace sd {
namespace {

constexpr int kRowsPerBlock = 4;  // 4 waves per 256-thread workgroup, one row each

// 16-byte vector path: row_vecs = row_elems / 8 uint4 per row; strides in uint4 units.
__global__ __launch_bounds__(256) void store_kvcache_vec(const uint4* __restrict__ key, int64_t key_stride,
                                                         const uint4* __restrict__ value, int64_t value_stride,
                                                         uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
                                                         const int32_t* __restrict__ slots, int32_t num_tokens,
                                                         int32_t row_vecs, int64_t num_slots) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t idx = (int64_t)blockIdx.x * kRowsPerBlock + wave;
  if (idx >= num_tokens) return;
  const int64_t slot = slots[idx];
  const uint4* ksrc = key + idx * key_stride;
  const uint4* vsrc = value + idx * value_stride;
  // The first step's loads go out with the slot's (the source row exists whatever the slot), so the row's
  // latency is one memory round trip, not two.
  int i = lane;
  const bool two = i + kWave < row_vecs, one = i < row_vecs;
  uint4 k0{}, k1{}, v0{}, v1{};
  if (two) {
    k0 = ksrc[i];
    k1 = ksrc[i + kWave];
    v0 = vsrc[i];
    v1 = vsrc[i + kWave];
  } else if (one) {
    k0 = ksrc[i];
    v0 = vsrc[i];
  }
  if (slot < 0 || slot >= num_slots) return;
  uint4* kdst = k_cache + slot * row_vecs;
  uint4* vdst = v_cache + slot * row_vecs;
  if (two) {
    kdst[i] = k0;
    kdst[i + kWave] = k1;
    vdst[i] = v0;
    vdst[i + kWave] = v1;
  } else if (one) {
    kdst[i] = k0;
    vdst[i] = v0;
  }
  i += 2 * kWave;
  // Two vectors of each tensor per lane per step keeps four 16-B loads in flight before the stores.
  for (; i + kWave < row_vecs; i += 2 * kWave) {
    uint4 k0 = ksrc[i], k1 = ksrc[i + kWave];
    uint4 v0 = vsrc[i], v1 = vsrc[i + kWave];
    kdst[i] = k0;
    kdst[i + kWave] = k1;
    vdst[i] = v0;
    vdst[i + kWave] = v1;
  }
  for (; i < row_vecs; i += kWave) {
    uint4 k0 = ksrc[i], v0 = vsrc[i];
    kdst[i] = k0;
    vdst[i] = v0;
  }
}

// Element path for rows or strides that are not 16-byte aligned.
__global__ __launch_bounds__(256) void store_kvcache_elem(const uint16_t* __restrict__ key, int64_t key_stride,
                                                          const uint16_t* __restrict__ value, int64_t value_stride,
                                                          uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                                                          const int32_t* __restrict__ slots, int32_t num_tokens,
                                                          int32_t row_elems, int64_t num_slots) {
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t idx = (int64_t)blockIdx.x * kRowsPerBlock + wave;
  if (idx >= num_tokens) return;
  const int64_t slot = slots[idx];
  if (slot < 0 || slot >= num_slots) return;
  for (int i = lane; i < row_elems; i += kWave) {
    k_cache[slot * row_elems + i] = key[idx * key_stride + i];
    v_cache[slot * row_elems + i] = value[idx * value_stride + i];
  }
}

}  // namespace
}  // namespace sd

using namespace sd;

extern "C" int sd_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                int64_t value_row_stride, void* k_cache, void* v_cache, int64_t num_slots,
                                const int32_t* slot_mapping, int32_t num_tokens, int32_t num_kv_heads,
                                int32_t head_dim, void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_slots < 0)
    return fail(kBadArgument, "sd_store_kvcache: bad sizes (tokens %d, kv heads %d, head_dim %d, slots %lld)",
                num_tokens, num_kv_heads, head_dim, (long long)num_slots);
  if (num_tokens == 0) return kOk;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(kBadArgument, "sd_store_kvcache: null pointer");
  const int32_t row_elems = num_kv_heads * head_dim;
  if (key_row_stride < row_elems || value_row_stride < row_elems)
    return fail(kBadArgument, "sd_store_kvcache: row stride smaller than num_kv_heads*head_dim");
  const dim3 grid((num_tokens + kRowsPerBlock - 1) / kRowsPerBlock), block(kRowsPerBlock * kWave);
  hipStream_t s = (hipStream_t)stream;
  const bool vec = row_elems % 8 == 0 && key_row_stride % 8 == 0 && value_row_stride % 8 == 0 &&
                   ((uintptr_t)key | (uintptr_t)value | (uintptr_t)k_cache | (uintptr_t)v_cache) % 16 == 0;
  if (vec) {
    hipLaunchKernelGGL(store_kvcache_vec, grid, block, 0, s, (const uint4*)key, key_row_stride / 8,
                       (const uint4*)value, value_row_stride / 8, (uint4*)k_cache, (uint4*)v_cache, slot_mapping,
                       num_tokens, row_elems / 8, num_slots);
  } else {
    hipLaunchKernelGGL(store_kvcache_elem, grid, block, 0, s, (const uint16_t*)key, key_row_stride,
                       (const uint16_t*)value, value_row_stride, (uint16_t*)k_cache, (uint16_t*)v_cache,
                       slot_mapping, num_tokens, row_elems, num_slots);
  }
  return check_launch("sd_store_kvcache");
}
