// LM head over the vocabulary without full logits (the consumer of the final norm's output):
// the per-chunk row kernel and the finalize kernel of the vocabulary-streamed head.  Replace
// head_chunk_kernel / head_finalize_kernel (solution/k_head.py:50-161); the two GEMMs of each
// chunk (logits = Y E_c^T, acc += P E_c in fp32) run on the fp16-weight GEMM entry points.
//
// Per row r, over vocabulary chunks [v0, v0 + vc) in order, state[r] = (m, s, t, argmax, x_t):
//   pass 1  m_c = max_j x_j, a_c = the first j reaching it, x_t = x[target - v0] if in the chunk
//   merge   m' = max(m, m_c); s' = s e^(m - m') + s_c e^(m_c - m');
//           t' = [s > 0] e^(m - m') (t + s (m - m')) + e^(m_c - m') (t_c + s_c (m_c - m'))
//           with s_c = sum e^(x - m_c), t_c = sum e^(x - m_c) (x - m_c); argmax moves only when
//           m_c > m (ties keep the earlier index)
//   pass 2  for rows with a target (r < n_lab): P = p_scale e^(x - m_c) e^(m_c - m') in place,
//           0 in the target's column; the row's fp32 gradient accumulator is rescaled by
//           e^(m - m') when that is below 1
// finalize: lse = m + log s, entropy = log s - t / s, loss = lse - x_t, hit = [argmax == target],
//   dY[perm[r]] = fp16(out_scale (acc / (p_scale s) + (e^(x_t - lse) - 1) E_t)) (zero without a
//   target).  Natural exp and log, fp32, every product and sum rounded on its own.
#include "dk_common.h"

namespace {

constexpr int kHThreads = 256;
constexpr int kStateW = 8;   // m, s, t, argmax, x_t, pad

// sum / max over the workgroup (fixed order: lanes by butterfly, then waves in order)
__device__ __forceinline__ float wg_reduce(float v, bool is_max, float* red) {
#pragma unroll
  for (int x = 32; x > 0; x >>= 1) {
    const float o = __shfl_xor(v, x);
    v = is_max ? fmaxf(v, o) : __fadd_rn(v, o);
  }
  const int w = threadIdx.x >> 6;
  __syncthreads();   // red is free
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < kHThreads / 64; ++i) r = is_max ? fmaxf(r, red[i]) : __fadd_rn(r, red[i]);
  return r;
}

__device__ __forceinline__ int wg_min_int(int v, int* red) {
#pragma unroll
  for (int x = 32; x > 0; x >>= 1) v = min(v, __shfl_xor(v, x));
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  int r = red[0];
#pragma unroll
  for (int i = 1; i < kHThreads / 64; ++i) r = min(r, red[i]);
  return r;
}

__global__ __launch_bounds__(kHThreads) void head_chunk_kernel(
    f16* __restrict__ logits, const int32_t* __restrict__ tgt, float* __restrict__ state,
    float* __restrict__ acc, int64_t n_lab, int64_t vc, int64_t v0, float p_scale, int64_t d) {
  const int64_t r = blockIdx.x;
  f16* row = logits + r * vc;
  __shared__ float redf[kHThreads / 64];
  __shared__ int redi[kHThreads / 64];
  const int64_t tloc = (int64_t)tgt[r] - v0;
  const bool in_chunk = tloc >= 0 && tloc < vc;
  // pass 1: this thread's pieces j = tid + 256 i (8 halves each), columns in increasing order
  float best = -INFINITY, xt = 0.0f;
  int best_i = INT32_MAX;
  for (int64_t j = threadIdx.x; 8 * j < vc; j += kHThreads) {
    const f16x8 x = *reinterpret_cast<const f16x8*>(row + 8 * j);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float xv = (float)x[e];
      const int col = (int)(8 * j + e);
      if (xv > best) {
        best = xv;
        best_i = col;
      }
      if (col == tloc) xt = xv;
    }
  }
  const float mc = wg_reduce(best, true, redf);
  const int ac = wg_min_int(best == mc ? best_i : INT32_MAX, redi);
  const float xt_c = wg_reduce(xt, false, redf);   // exactly x[tloc]: one thread holds it, the rest 0
  float* st = state + r * kStateW;
  const float m = st[0], s = st[1], tt = st[2], am = st[3], xto = st[4];
  const float m_new = fmaxf(m, mc);
  const float a_old = expf(__fsub_rn(m, m_new));   // 0 on the first chunk (m = -inf)
  const float a_new = expf(__fsub_rn(mc, m_new));
  const bool sup = r < n_lab;
  const float pmul = __fmul_rn(a_new, p_scale);
  // pass 2 (every pass-1 read of the row is ordered before these writes by the reductions' barriers)
  float as = 0.0f, at = 0.0f;
  for (int64_t j = threadIdx.x; 8 * j < vc; j += kHThreads) {
    const f16x8 x = *reinterpret_cast<const f16x8*>(row + 8 * j);
    f16x8 p;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float z = __fsub_rn((float)x[e], mc);
      const float ev = expf(z);
      as = __fadd_rn(as, ev);
      at = __fadd_rn(at, __fmul_rn(ev, z));
      p[e] = (int64_t)(8 * j + e) == tloc ? (f16)0.0f : (f16)__fmul_rn(ev, pmul);
    }
    if (sup) *reinterpret_cast<f16x8*>(row + 8 * j) = p;
  }
  const float sc = wg_reduce(as, false, redf);
  const float tc = wg_reduce(at, false, redf);
  if (threadIdx.x == 0) {
    const float s_new = __fadd_rn(__fmul_rn(s, a_old), __fmul_rn(sc, a_new));
    const float t_old = s > 0.0f ? __fmul_rn(a_old, __fadd_rn(tt, __fmul_rn(s, __fsub_rn(m, m_new))))
                                 : 0.0f;
    const float t_new = __fadd_rn(t_old, __fmul_rn(a_new, __fadd_rn(tc, __fmul_rn(sc, __fsub_rn(mc, m_new)))));
    st[0] = m_new;
    st[1] = s_new;
    st[2] = t_new;
    st[3] = mc > m ? (float)(ac + v0) : am;
    st[4] = in_chunk ? xt_c : xto;
  }
  if (sup && a_old < 1.0f) {
    float* arow = acc + r * d;
    for (int64_t i = threadIdx.x; 4 * i < d; i += kHThreads) {
      f32x4 a = *reinterpret_cast<const f32x4*>(arow + 4 * i);
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = __fmul_rn(a[e], a_old);
      *reinterpret_cast<f32x4*>(arow + 4 * i) = a;
    }
  }
}

__global__ __launch_bounds__(kHThreads) void head_finalize_kernel(
    const float* __restrict__ state, const int32_t* __restrict__ tgt, const int32_t* __restrict__ perm,
    const float* __restrict__ acc, const f16* __restrict__ et, float* __restrict__ stats,
    f16* __restrict__ dy, int64_t n_lab, float out_scale, float inv_p_scale, int64_t d) {
  const int64_t r = blockIdx.x;
  const float* st = state + r * kStateW;
  const float m = st[0], s = st[1], tt = st[2], am = st[3], xt = st[4];
  const float log_s = logf(s);
  const float lse = __fadd_rn(m, log_s);
  const int t = tgt[r];
  if (threadIdx.x == 0) {
    const bool valid = t >= 0;
    stats[r * 4 + 0] = valid ? __fsub_rn(lse, xt) : 0.0f;
    stats[r * 4 + 1] = __fsub_rn(log_s, __fdiv_rn(tt, s));
    stats[r * 4 + 2] = valid && am == (float)t ? 1.0f : 0.0f;
    stats[r * 4 + 3] = lse;
  }
  const int64_t dst = perm[r];
  if (dst < 0 || dst >= (int64_t)gridDim.x) return;   // not a row of this batch: nothing written
  f16* out = dy + dst * d;
  if (r < n_lab) {
    const float pt1 = __fsub_rn(expf(__fsub_rn(xt, lse)), 1.0f);
    const float q = __fdiv_rn(inv_p_scale, s);
    const float* arow = acc + r * d;
    const f16* erow = et + r * d;
    for (int64_t i = threadIdx.x; 4 * i < d; i += kHThreads) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(arow + 4 * i);
      const f16x4 e = *reinterpret_cast<const f16x4*>(erow + 4 * i);
      f16x4 o;
#pragma unroll
      for (int k = 0; k < 4; ++k)
        o[k] = (f16)__fmul_rn(__fadd_rn(__fmul_rn(a[k], q), __fmul_rn(pt1, (float)e[k])), out_scale);
      *reinterpret_cast<f16x4*>(out + 4 * i) = o;
    }
  } else {
    for (int64_t i = threadIdx.x; 4 * i < d; i += kHThreads)
      *reinterpret_cast<f16x4*>(out + 4 * i) = f16x4{(f16)0.0f, (f16)0.0f, (f16)0.0f, (f16)0.0f};
  }
}

}  // namespace

extern "C" int dk_head_chunk(void* logits, const int32_t* tgt_sorted, float* state, float* acc,
                             int64_t n_rows, int64_t n_lab, int64_t vc, int64_t v0, float p_scale,
                             int64_t d, hipStream_t stream) {
  // one workgroup per row (the grid's x limit); the argmax index is kept as an fp32 in the state,
  // exact for every column below 2^24
  if (n_rows < 0 || n_rows > INT32_MAX || n_lab < 0 || n_lab > n_rows || vc <= 0 || vc % 8 ||
      vc > INT32_MAX / 2 || v0 < 0 || v0 + vc > (int64_t{1} << 24) || d <= 0 || d % 4)
    return DK_ERR_INVALID;
  if (n_rows == 0) return 0;
  if (!logits || !tgt_sorted || !state || (n_lab > 0 && !acc)) return DK_ERR_INVALID;
  if (!dk_aligned(logits, 16) || !dk_aligned(state, 4) || !dk_aligned(tgt_sorted, 4) ||
      (acc && !dk_aligned(acc, 16)))
    return DK_ERR_ALIGN;
  hipLaunchKernelGGL(head_chunk_kernel, dim3((unsigned)n_rows), dim3(kHThreads), 0, stream,
                     (f16*)logits, tgt_sorted, state, acc, n_lab, vc, v0, p_scale, d);
  DK_CHECK_LAUNCH();
  return 0;
}

extern "C" int dk_head_finalize(const float* state, const int32_t* tgt_sorted, const int32_t* perm,
                                const float* acc, const void* e_target, float* stats, void* dy,
                                int64_t n_rows, int64_t n_lab, float out_scale, float inv_p_scale,
                                int64_t d, hipStream_t stream) {
  if (n_rows < 0 || n_rows > INT32_MAX || n_lab < 0 || n_lab > n_rows || d <= 0 || d % 4)
    return DK_ERR_INVALID;
  if (n_rows == 0) return 0;
  if (!state || !tgt_sorted || !perm || !stats || !dy || (n_lab > 0 && (!acc || !e_target)))
    return DK_ERR_INVALID;
  if (!dk_aligned(dy, 8) || (acc && !dk_aligned(acc, 16)) || (e_target && !dk_aligned(e_target, 8)))
    return DK_ERR_ALIGN;
  hipLaunchKernelGGL(head_finalize_kernel, dim3((unsigned)n_rows), dim3(kHThreads), 0, stream,
                     state, tgt_sorted, perm, acc, (const f16*)e_target, stats, (f16*)dy, n_lab,
                     out_scale, inv_p_scale, d);
  DK_CHECK_LAUNCH();
  return 0;
}
