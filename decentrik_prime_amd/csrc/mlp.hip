// Gated SiLU of the Qwen2 MLP on the fused [gate | up] rows, and the stock path's example SwiGLU.
//
// gated_silu (replaces solution/k_mlp.py:20-63): 2-D grid (row, 2048-column tile); a thread
// takes 8 consecutive columns with 16-byte loads and stores when the row layout allows it (inter
// a multiple of 8, 16-byte aligned bases), one column at a time otherwise.  fp32 math:
//   forward   act = fp16(g / (1 + exp(-g)) * u)
//   backward  e = 1 + exp(-g), sig = 1 / e, silu = g / e
//             gu <- [fp16((da * u) * sig * (1 + g * (1 - sig))) | fp16(da * silu)]
#include "dk_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kVec = 8;
constexpr int kColsPerBlock = kThreads * kVec;

__device__ __forceinline__ float silu_of(float g, float* e_out) {
  const float e = 1.0f + __expf(-g);
  *e_out = e;
  return g / e;
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void gated_silu_fwd_kernel(const f16* __restrict__ gu,
                                                                  f16* __restrict__ act,
                                                                  int64_t inter) {
  const int64_t row = blockIdx.x;
  const f16* g_row = gu + row * 2 * inter;
  const f16* u_row = g_row + inter;
  f16* a_row = act + row * inter;
  const int64_t c0 = (int64_t)blockIdx.y * kColsPerBlock + (int64_t)threadIdx.x * kVec;
  if (VEC) {
    if (c0 >= inter) return;
    const f16x8 g = *reinterpret_cast<const f16x8*>(g_row + c0);
    const f16x8 u = *reinterpret_cast<const f16x8*>(u_row + c0);
    f16x8 o;
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      float e;
      const float s = silu_of((float)g[i], &e);
      o[i] = dk_h(s * (float)u[i]);
    }
    *reinterpret_cast<f16x8*>(a_row + c0) = o;
  } else {
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      const int64_t c = c0 + i;
      if (c < inter) {
        float e;
        const float s = silu_of((float)g_row[c], &e);
        a_row[c] = dk_h(s * (float)u_row[c]);
      }
    }
  }
}

__device__ __forceinline__ void gated_silu_grad(float g, float u, float da, f16* dg, f16* du) {
  float e;
  const float silu = silu_of(g, &e);
  const float sig = 1.0f / e;
  *du = dk_h(da * silu);
  *dg = dk_h((da * u) * sig * (1.0f + g * (1.0f - sig)));
}

template <bool VEC>
__global__ __launch_bounds__(kThreads) void gated_silu_bwd_kernel(f16* __restrict__ gu,
                                                                  const f16* __restrict__ dact,
                                                                  int64_t inter) {
  const int64_t row = blockIdx.x;
  f16* g_row = gu + row * 2 * inter;
  f16* u_row = g_row + inter;
  const f16* d_row = dact + row * inter;
  const int64_t c0 = (int64_t)blockIdx.y * kColsPerBlock + (int64_t)threadIdx.x * kVec;
  if (VEC) {
    if (c0 >= inter) return;
    const f16x8 g = *reinterpret_cast<const f16x8*>(g_row + c0);
    const f16x8 u = *reinterpret_cast<const f16x8*>(u_row + c0);
    const f16x8 d = *reinterpret_cast<const f16x8*>(d_row + c0);
    f16x8 og, ou;
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      f16 a, b;
      gated_silu_grad((float)g[i], (float)u[i], (float)d[i], &a, &b);
      og[i] = a;
      ou[i] = b;
    }
    *reinterpret_cast<f16x8*>(g_row + c0) = og;
    *reinterpret_cast<f16x8*>(u_row + c0) = ou;
  } else {
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
      const int64_t c = c0 + i;
      if (c < inter) {
        f16 a, b;
        gated_silu_grad((float)g_row[c], (float)u_row[c], (float)d_row[c], &a, &b);
        g_row[c] = a;
        u_row[c] = b;
      }
    }
  }
}

// Example SwiGLU (solution/swiglu.py:15-37): flat, out-of-place.
__global__ __launch_bounds__(kThreads) void swiglu_fwd_kernel(const f16* __restrict__ gate,
                                                              const f16* __restrict__ up,
                                                              f16* __restrict__ out, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const float g = (float)gate[i];
  const float sig = 1.0f / (1.0f + __expf(-g));
  out[i] = dk_h(g * sig * (float)up[i]);
}

__global__ __launch_bounds__(kThreads) void swiglu_bwd_kernel(
    const f16* __restrict__ grad, const f16* __restrict__ gate, const f16* __restrict__ up,
    f16* __restrict__ dgate, f16* __restrict__ dup, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= n) return;
  const float gr = (float)grad[i];
  const float g = (float)gate[i];
  const float u = (float)up[i];
  const float sig = 1.0f / (1.0f + __expf(-g));
  dup[i] = dk_h(gr * g * sig);
  dgate[i] = dk_h(gr * u * sig * (1.0f + g * (1.0f - sig)));
}

bool vec_ok(const void* a, const void* b, int64_t inter) {
  return inter % kVec == 0 && dk_aligned(a, 16) && dk_aligned(b, 16);
}

}  // namespace

extern "C" int dk_gated_silu_fwd(const void* gu, void* act, int64_t n_rows, int64_t inter,
                                 hipStream_t stream) {
  if (n_rows < 0 || inter <= 0 || inter > (int64_t)kColsPerBlock * 65535) return DK_ERR_INVALID;
  if (n_rows == 0) return 0;
  if (!gu || !act) return DK_ERR_INVALID;
  dim3 grid((unsigned)n_rows, (unsigned)((inter + kColsPerBlock - 1) / kColsPerBlock));
  if (vec_ok(gu, act, inter))
    hipLaunchKernelGGL(gated_silu_fwd_kernel<true>, grid, dim3(kThreads), 0, stream,
                       (const f16*)gu, (f16*)act, inter);
  else
    hipLaunchKernelGGL(gated_silu_fwd_kernel<false>, grid, dim3(kThreads), 0, stream,
                       (const f16*)gu, (f16*)act, inter);
  DK_CHECK_LAUNCH();
  return 0;
}

extern "C" int dk_gated_silu_bwd(void* gu, const void* dact, int64_t n_rows, int64_t inter,
                                 hipStream_t stream) {
  if (n_rows < 0 || inter <= 0 || inter > (int64_t)kColsPerBlock * 65535) return DK_ERR_INVALID;
  if (n_rows == 0) return 0;
  if (!gu || !dact) return DK_ERR_INVALID;
  dim3 grid((unsigned)n_rows, (unsigned)((inter + kColsPerBlock - 1) / kColsPerBlock));
  if (vec_ok(gu, dact, inter))
    hipLaunchKernelGGL(gated_silu_bwd_kernel<true>, grid, dim3(kThreads), 0, stream, (f16*)gu,
                       (const f16*)dact, inter);
  else
    hipLaunchKernelGGL(gated_silu_bwd_kernel<false>, grid, dim3(kThreads), 0, stream, (f16*)gu,
                       (const f16*)dact, inter);
  DK_CHECK_LAUNCH();
  return 0;
}

extern "C" int dk_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n,
                             hipStream_t stream) {
  if (n < 0) return DK_ERR_INVALID;
  if (n == 0) return 0;
  if (!gate || !up || !out) return DK_ERR_INVALID;
  hipLaunchKernelGGL(swiglu_fwd_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, (const f16*)gate, (const f16*)up, (f16*)out, n);
  DK_CHECK_LAUNCH();
  return 0;
}

extern "C" int dk_swiglu_bwd(const void* grad, const void* gate, const void* up, void* dgate,
                             void* dup, int64_t n, hipStream_t stream) {
  if (n < 0) return DK_ERR_INVALID;
  if (n == 0) return 0;
  if (!grad || !gate || !up || !dgate || !dup) return DK_ERR_INVALID;
  hipLaunchKernelGGL(swiglu_bwd_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, (const f16*)grad, (const f16*)gate,
                     (const f16*)up, (f16*)dgate, (f16*)dup, n);
  DK_CHECK_LAUNCH();
  return 0;
}
