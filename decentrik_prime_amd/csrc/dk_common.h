// Shared definitions for the gfx950 kernels of the NF4 QLoRA linear path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dk.h"

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Second-level block: 256 first-level blocks of 64 weights.
#define DK_QBLOCK 64
#define DK_QBLOCK2 256
#define DK_ELEMS_PER_SB (DK_QBLOCK * DK_QBLOCK2)

#define DK_CHECK_LAUNCH()                       \
  do {                                          \
    hipError_t e_ = hipGetLastError();          \
    if (e_ != hipSuccess) return (int)e_;       \
  } while (0)

static inline bool dk_aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// fp32 -> fp16, round to nearest even (v_cvt_f16_f32 under the default round mode).
// fp16 of an fp32 value, rounded the way the reference rounds: the fp32 result of the producing
// multiply or add first, then fp16.  The empty asm keeps the compiler from folding that multiply
// or add and this conversion into one v_fma_mix*_f16, which rounds the exact result straight to
// fp16 and differs in the last fp16 bit for about 1 input in 10^4.
__device__ __forceinline__ f16 dk_h(float x) {
  asm("" : "+v"(x));
  return (f16)x;
}

// Logistic parts of the gated SiLU for the GEMM epilogues: e = 1 + exp(-g), sig = 1/e and
// silu = g/e through one hardware reciprocal (v_rcp_f32, about 1 ulp) instead of two IEEE
// divisions; far below the fp16 rounding of the results.
__device__ __forceinline__ void dk_silu_parts(float g, float* sig, float* silu) {
  const float r = __builtin_amdgcn_rcpf(1.0f + __expf(-g));
  *sig = r;
  *silu = g * r;
}

// Pack two fp16 into one dword, lower address in the low half.
__device__ __forceinline__ uint32_t dk_pack2(f16 lo, f16 hi) {
  f16x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, v);
}

// absmax of first-level block q: fp32(fp32(code2[c] * scale2) + offset2), product and sum rounded
// separately.  Kernels that include this header are compiled with -ffp-contract=off.
__device__ __forceinline__ float dk_absmax(float c2, float s2, float o2) {
  float first = __fmul_rn(c2, s2);
  return __fadd_rn(first, o2);
}
