// Shared definitions for the spec-decode attention / verify kernels (CDNA4, gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sd {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Status codes returned by every C-ABI entry point (0 = success).
enum Status : int {
  kOk = 0,
  kBadArgument = 1,
  kUnsupported = 2,
  kWorkspaceTooSmall = 3,
  kLaunchFailed = 4,
};

// Records a formatted message for sd_last_error(); returns `code` for `return fail(...)` chains.
int fail(int code, const char* fmt, ...);
// Checks hipGetLastError() after a launch; returns kOk or kLaunchFailed (message recorded).
int check_launch(const char* what);

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet (same rounding as torch's bfloat16 cast).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __builtin_bit_cast(float, ((uint32_t)h) << 16);
}

// Two fp32 -> one dword holding two bf16 (low half = a).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)f32_to_bf16_bits(a) | ((uint32_t)f32_to_bf16_bits(b) << 16);
}

// Compiler + LDS ordering point for wave-private LDS reuse: waits for this wave's outstanding LDS
// operations and keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_wave_fence() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// 2^x with the hardware v_exp_f32.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane exchange with the gfx950 lane-swap instructions instead of LDS permutes.
// v_permlane16_swap(a, b) exchanges the odd 16-lane rows of a with the even rows of b (v_permlane32_swap:
// upper half of a with lower half of b), so with a = b = x every lane ends up holding x of itself and of
// its partner. Written as inline asm because
// the compiler's builtin does not keep the second register of the pair; the s_nops cover the VALU-write /
// permlane-read hazard on both sides.
__device__ __forceinline__ void swap16(uint32_t& a, uint32_t& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void swap32(uint32_t& a, uint32_t& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}

// true if (v, i) should replace (bv, bi) under torch.argmax order: NaN largest, then value, then lower index.
__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  const bool vn = v != v, bn = bv != bv;
  if (vn || bn) return vn && (!bn || i < bi);
  return v > bv || (v == bv && i < bi);
}

// Two fp32 -> packed bf16 (v_cvt_pk_bf16_f32, round to nearest even).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ds_read_b64_tr_b16 at LDS byte address `addr` + OFF, as inline asm: with the builtin form the compiler
// waits for every outstanding vector-memory load (vmcnt(0)) before each read. The caller waits
// lgkmcnt(0) (tied to the results) before using them.
template <int OFF>
__device__ __forceinline__ u32x2 ds_read_tr16(uint32_t addr) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF) : "memory");
  return r;
}

// ds_read_b128 at LDS byte address `addr`, as inline asm (batched reads with one tied wait; see above).
__device__ __forceinline__ bf16x8 ds_read_b128(uint32_t addr) {
  bf16x8 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr) : "memory");
  return r;
}

// CUs of the device that runs `stream` (the null stream: the current device's), queried once per device.
// Host code only.
inline int cu_count(hipStream_t stream) {
  static int cached[64];  // per device; 0 until first queried (a racing second query stores the same value)
  hipDevice_t dev = 0;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess && hipGetDevice(&dev) != hipSuccess) return 256;
  if (dev < 0 || dev >= 64) return 256;
  int cus = __atomic_load_n(&cached[dev], __ATOMIC_RELAXED);
  if (!cus) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    __atomic_store_n(&cached[dev], cus, __ATOMIC_RELAXED);
  }
  return cus;
}

}  // namespace sd
