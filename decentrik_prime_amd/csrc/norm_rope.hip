// The producer and the consumer around the LoRA'd q/v linear (gfx950): the fused residual add +
// RMSNorm that also emits the two dropout-masked LoRA inputs, its backward with the LoRA input
// gradients, and the QKV epilogue (LoRA add + rotary embedding, and its transpose with the GQA
// partial sums).  Replace solution/k_norm.py:29-88 and solution/k_rope.py:23-104.
//
// Both are HBM-bound row kernels: one wave per token row, 64 lanes over the row in 16-byte
// vectors, four rows per 256-thread workgroup; all of a row's loads are issued before its first
// use.  Every product and sum is rounded to fp32 on its own (-ffp-contract=off), as the
// reference's kernels (compiled with fp fusion off for the QKV epilogue) round; the row sums are
// a lane-order sum followed by a butterfly across the wave, a different order from the
// reference's tree, within the reference tests' tolerances.
#include "dk_common.h"

namespace {

constexpr int kRowThreads = 256;
constexpr int kRowsPerBlock = kRowThreads / 64;
constexpr int kBatch = 4;     // QKV epilogue tasks per lane whose loads are in flight together
constexpr int kGinBatch = 6;  // GQA partials per KV head whose loads are in flight together

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ f32x4 load_h4(const f16* p) {
  const f16x4 h = *reinterpret_cast<const f16x4*>(p);
  return f32x4{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
}

__device__ __forceinline__ void store_h4(f16* p, const f32x4& v) {
  *reinterpret_cast<f16x4*>(p) = f16x4{dk_h(v[0]), dk_h(v[1]), dk_h(v[2]), dk_h(v[3])};
}

__device__ __forceinline__ uint32_t load_mask4(const uint8_t* p) {
  return *reinterpret_cast<const uint32_t*>(p);
}

__device__ __forceinline__ bool kept(uint32_t m4, int e) { return ((m4 >> (8 * e)) & 0xffu) != 0; }

// ---------------------------------------------------------------------------------------------
// RMSNorm forward (solution/k_norm.py:38-58).  Lane l of a row handles elements 256 k + 4 l .. +3
// for k < ceil(D / 256); KMAX bounds the chunks held in registers.
template <int KMAX>
__global__ __launch_bounds__(kRowThreads) void rms_fwd_kernel(
    const float* __restrict__ x, const f16* __restrict__ delta, float* __restrict__ xout,
    const float* __restrict__ w, f16* __restrict__ y, float* __restrict__ rstd,
    f16* __restrict__ xq, f16* __restrict__ xv, const uint8_t* __restrict__ mq,
    const uint8_t* __restrict__ mv, int64_t n_rows, int d, float eps, float keep_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int64_t off = row * d;
  // every load of the row is issued before the reduction, so the row costs one memory latency
  f32x4 h[KMAX], wv[KMAX];
  uint32_t kq[KMAX], kv[KMAX];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int e = 256 * k + 4 * lane;
    if (e < d) {
      h[k] = *reinterpret_cast<const f32x4*>(x + off + e);
      wv[k] = *reinterpret_cast<const f32x4*>(w + e);
      if (xq) {
        kq[k] = load_mask4(mq + off + e);
        kv[k] = load_mask4(mv + off + e);
      }
      if (delta) {
        const f32x4 dl = load_h4(delta + off + e);
#pragma unroll
        for (int i = 0; i < 4; ++i) h[k][i] = __fadd_rn(h[k][i], dl[i]);
      }
      if (xout) *reinterpret_cast<f32x4*>(xout + off + e) = h[k];
#pragma unroll
      for (int i = 0; i < 4; ++i) ss = __fadd_rn(ss, __fmul_rn(h[k][i], h[k][i]));
    }
  }
  const float ms = __fmul_rn(wave_sum(ss), 1.0f / (float)d);
  const float r = rsqrtf(__fadd_rn(ms, eps));
  if (lane == 0) rstd[row] = r;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int e = 256 * k + 4 * lane;
    if (e >= d) continue;
    f32x4 yv;
#pragma unroll
    for (int i = 0; i < 4; ++i) yv[i] = __fmul_rn(wv[k][i], __fmul_rn(h[k][i], r));
    if (y) store_h4(y + off + e, yv);
    if (xq) {
      f32x4 a, b;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ys = __fmul_rn(yv[i], keep_scale);
        a[i] = kept(kq[k], i) ? ys : 0.0f;
        b[i] = kept(kv[k], i) ? ys : 0.0f;
      }
      store_h4(xq + off + e, a);
      store_h4(xv + off + e, b);
    }
  }
}

// RMSNorm backward (solution/k_norm.py:61-88): dy = fp16 grad * gscale + the masked LoRA input
// grads, dx = rstd (w dy - xhat mean(w dy xhat)) [+ dres]; out may alias dres.
template <int KMAX, bool DY32>
__global__ __launch_bounds__(kRowThreads) void rms_bwd_kernel(
    const void* __restrict__ dyp, const float* __restrict__ gscale, const float* __restrict__ x,
    const f16* __restrict__ delta, const float* __restrict__ w, const float* __restrict__ rstd,
    const float* dres, float* out, const f16* __restrict__ lq, const f16* __restrict__ lv,
    f16* __restrict__ out16, const uint8_t* __restrict__ mq, const uint8_t* __restrict__ mv,
    int64_t n_rows, int d, float keep_scale) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int64_t off = row * d;
  const float gs = *gscale;
  const float r = rstd[row];
  f32x4 g[KMAX], xh[KMAX], rv[KMAX];
  float cs = 0.0f;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int e = 256 * k + 4 * lane;
    if (e >= d) continue;
    f32x4 dy = DY32 ? *reinterpret_cast<const f32x4*>(static_cast<const float*>(dyp) + off + e)
                    : load_h4(static_cast<const f16*>(dyp) + off + e);
#pragma unroll
    for (int i = 0; i < 4; ++i) dy[i] = __fmul_rn(dy[i], gs);
    if (lq) {
      const uint32_t kq = load_mask4(mq + off + e), kv = load_mask4(mv + off + e);
      const f32x4 a = load_h4(lq + off + e), b = load_h4(lv + off + e);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dy[i] = __fadd_rn(dy[i], kept(kq, i) ? __fmul_rn(a[i], keep_scale) : 0.0f);
        dy[i] = __fadd_rn(dy[i], kept(kv, i) ? __fmul_rn(b[i], keep_scale) : 0.0f);
      }
    }
    f32x4 xv = *reinterpret_cast<const f32x4*>(x + off + e);
    if (delta) {
      const f32x4 dl = load_h4(delta + off + e);
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[i] = __fadd_rn(xv[i], dl[i]);
    }
    const f32x4 wv = *reinterpret_cast<const f32x4*>(w + e);
    if (dres) rv[k] = *reinterpret_cast<const f32x4*>(dres + off + e);   // before the reduction
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xh[k][i] = __fmul_rn(xv[i], r);
      g[k][i] = __fmul_rn(dy[i], wv[i]);
      cs = __fadd_rn(cs, __fmul_rn(g[k][i], xh[k][i]));
    }
  }
  const float c = __fmul_rn(wave_sum(cs), 1.0f / (float)d);
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int e = 256 * k + 4 * lane;
    if (e >= d) continue;
    f32x4 dx;
#pragma unroll
    for (int i = 0; i < 4; ++i) dx[i] = __fmul_rn(__fsub_rn(g[k][i], __fmul_rn(xh[k][i], c)), r);
    if (dres) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dx[i] = __fadd_rn(dx[i], rv[k][i]);
    }
    *reinterpret_cast<f32x4*>(out + off + e) = dx;
    if (out16) store_h4(out16 + off + e, dx);
  }
}

// ---------------------------------------------------------------------------------------------
// QKV epilogue forward (solution/k_rope.py:23-61), in place on a row of
// [q heads | k heads | v heads] x hd fp16.  Tasks of 4 consecutive pair indices j of one head
// (both halves, 8-byte accesses), then the v heads in 4-element pieces.
__global__ __launch_bounds__(kRowThreads) void qkv_epilogue_fwd_kernel(
    f16* qkv, const f16* __restrict__ lq, const f16* __restrict__ lv,
    const int32_t* __restrict__ pos, const float* __restrict__ cosv, const float* __restrict__ sinv,
    int64_t n_rows, float scale, int nq, int nkv, int hd) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int half = hd / 2, quads = half / 4;
  const int64_t p = pos[row];
  const float* cr = cosv + p * hd;
  const float* sr = sinv + p * hd;
  f16* base = qkv + row * (int64_t)(nq + 2 * nkv) * hd;
  const f16* lqr = lq + row * (int64_t)nq * hd;
  const f16* lvr = lv + row * (int64_t)nkv * hd;
  // query heads (LoRA add, rotate) and key heads (rotate): a lane's tasks t = lane + 64 i in
  // batches of kBatch, all loads of a batch issued before the first is used
  const int tasks = (nq + nkv) * quads;
  for (int t0 = 0; t0 < tasks; t0 += 64 * kBatch) {
    f32x4 x1[kBatch], x2[kBatch], a[kBatch], b[kBatch], c[kBatch], s[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= tasks) continue;
      const int head = t / quads, j = 4 * (t % quads);
      const f16* h1 = base + head * hd + j;
      x1[u] = load_h4(h1);
      x2[u] = load_h4(h1 + half);
      c[u] = *reinterpret_cast<const f32x4*>(cr + j);
      s[u] = *reinterpret_cast<const f32x4*>(sr + j);
      if (head < nq) {
        a[u] = load_h4(lqr + head * hd + j);
        b[u] = load_h4(lqr + head * hd + j + half);
      }
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= tasks) continue;
      const int head = t / quads, j = 4 * (t % quads);
      if (head < nq) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x1[u][i] = __fadd_rn(x1[u][i], __fmul_rn(a[u][i], scale));
          x2[u][i] = __fadd_rn(x2[u][i], __fmul_rn(b[u][i], scale));
        }
      }
      f32x4 o1, o2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o1[i] = __fsub_rn(__fmul_rn(x1[u][i], c[u][i]), __fmul_rn(x2[u][i], s[u][i]));
        o2[i] = __fadd_rn(__fmul_rn(x2[u][i], c[u][i]), __fmul_rn(x1[u][i], s[u][i]));
      }
      f16* h1 = base + head * hd + j;
      store_h4(h1, o1);
      store_h4(h1 + half, o2);
    }
  }
  // value heads: LoRA add
  f16* vb = base + (int64_t)(nq + nkv) * hd;
  const int vtasks = nkv * hd / 4;
  for (int t0 = 0; t0 < vtasks; t0 += 64 * kBatch) {
    f32x4 v[kBatch], a[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= vtasks) continue;
      v[u] = load_h4(vb + 4 * t);
      a[u] = load_h4(lvr + 4 * t);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= vtasks) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[u][i] = __fadd_rn(v[u][i], __fmul_rn(a[u][i], scale));
      store_h4(vb + 4 * t, v[u]);
    }
  }
}

template <typename T>
__device__ __forceinline__ f32x4 load4(const T* p) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const f32x4*>(p);
  } else {
    return load_h4(reinterpret_cast<const f16*>(p));
  }
}

// QKV epilogue backward (solution/k_rope.py:64-104): the transposed rotation of dq; the gin
// partials of each KV head summed in order, dk rotated back; fp16 out in the QKV layout.
template <typename T>
__global__ __launch_bounds__(kRowThreads) void qkv_epilogue_bwd_kernel(
    const T* __restrict__ dq, const T* __restrict__ dk, const T* __restrict__ dv,
    const int32_t* __restrict__ pos, const float* __restrict__ cosv, const float* __restrict__ sinv,
    f16* __restrict__ out, int64_t n_rows, int nq, int nkv, int hd, int gin) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const int half = hd / 2, quads = half / 4;
  const int64_t p = pos[row];
  const float* cr = cosv + p * hd;
  const float* sr = sinv + p * hd;
  f16* dst = out + row * (int64_t)(nq + 2 * nkv) * hd;
  const T* dqr = dq + row * (int64_t)nq * hd;
  const T* dkr = dk + row * (int64_t)nkv * gin * hd;
  const T* dvr = dv + row * (int64_t)nkv * gin * hd;
  // query heads: batches of kBatch tasks, all loads first
  const int qtasks = nq * quads;
  for (int t0 = 0; t0 < qtasks; t0 += 64 * kBatch) {
    f32x4 d1[kBatch], d2[kBatch], c[kBatch], s[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= qtasks) continue;
      const int head = t / quads, j = 4 * (t % quads);
      d1[u] = load4(dqr + head * hd + j);
      d2[u] = load4(dqr + head * hd + j + half);
      c[u] = *reinterpret_cast<const f32x4*>(cr + j);
      s[u] = *reinterpret_cast<const f32x4*>(sr + j);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= qtasks) continue;
      const int head = t / quads, j = 4 * (t % quads);
      f32x4 o1, o2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o1[i] = __fadd_rn(__fmul_rn(d1[u][i], c[u][i]), __fmul_rn(d2[u][i], s[u][i]));
        o2[i] = __fsub_rn(__fmul_rn(d2[u][i], c[u][i]), __fmul_rn(d1[u][i], s[u][i]));
      }
      store_h4(dst + head * hd + j, o1);
      store_h4(dst + head * hd + j + half, o2);
    }
  }
  // key heads: the gin partials summed in order (up to kGinBatch partials' loads in flight), then
  // the transposed rotation; value heads: the partials summed
  const int ktasks = nkv * quads;
  for (int t = lane; t < ktasks; t += 64) {
    const int hk = t / quads, j = 4 * (t % quads);
    const f32x4 c = *reinterpret_cast<const f32x4*>(cr + j);
    const f32x4 s = *reinterpret_cast<const f32x4*>(sr + j);
    f32x4 d1 = f32x4{0.0f, 0.0f, 0.0f, 0.0f}, d2 = d1;
    for (int g0 = 0; g0 < gin; g0 += kGinBatch) {
      f32x4 pa[kGinBatch], pb[kGinBatch];
#pragma unroll
      for (int u = 0; u < kGinBatch; ++u) {
        if (g0 + u >= gin) continue;
        const T* part = dkr + (int64_t)(hk * gin + g0 + u) * hd + j;
        pa[u] = load4(part);
        pb[u] = load4(part + half);
      }
#pragma unroll
      for (int u = 0; u < kGinBatch; ++u) {
        if (g0 + u >= gin) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          d1[i] = __fadd_rn(d1[i], pa[u][i]);
          d2[i] = __fadd_rn(d2[i], pb[u][i]);
        }
      }
    }
    f32x4 o1, o2;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o1[i] = __fadd_rn(__fmul_rn(d1[i], c[i]), __fmul_rn(d2[i], s[i]));
      o2[i] = __fsub_rn(__fmul_rn(d2[i], c[i]), __fmul_rn(d1[i], s[i]));
    }
    store_h4(dst + (nq + hk) * hd + j, o1);
    store_h4(dst + (nq + hk) * hd + j + half, o2);
  }
  f16* vdst = dst + (int64_t)(nq + nkv) * hd;
  for (int t = lane; t < nkv * hd / 4; t += 64) {
    const int hk = (4 * t) / hd, e = (4 * t) % hd;
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int g0 = 0; g0 < gin; g0 += kGinBatch) {
      f32x4 pa[kGinBatch];
#pragma unroll
      for (int u = 0; u < kGinBatch; ++u)
        if (g0 + u < gin) pa[u] = load4(dvr + (int64_t)(hk * gin + g0 + u) * hd + e);
#pragma unroll
      for (int u = 0; u < kGinBatch; ++u) {
        if (g0 + u >= gin) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], pa[u][i]);
      }
    }
    store_h4(vdst + 4 * t, acc);
  }
}

int grid_rows(int64_t n_rows) { return (int)((n_rows + kRowsPerBlock - 1) / kRowsPerBlock); }

}  // namespace

extern "C" int dk_rms_fwd(const float* x, const void* delta, float* xout, const float* w, void* y,
                          float* rstd, void* xq, void* xv, const uint8_t* mq, const uint8_t* mv,
                          int64_t n_rows, int64_t d, float eps, float keep_scale,
                          hipStream_t stream) {
  if (n_rows < 0 || d < 4 || d > 4096 || d % 4) return DK_ERR_INVALID;
  if (n_rows == 0) return 0;
  if (!x || !w || !rstd) return DK_ERR_INVALID;
  if ((xq == nullptr) != (xv == nullptr) || (xq && (!mq || !mv))) return DK_ERR_INVALID;
  if (!dk_aligned(x, 16) || !dk_aligned(w, 16) || (xout && !dk_aligned(xout, 16)) ||
      (delta && !dk_aligned(delta, 8)) || (y && !dk_aligned(y, 8)) ||
      (xq && (!dk_aligned(xq, 8) || !dk_aligned(xv, 8) || !dk_aligned(mq, 4) || !dk_aligned(mv, 4))))
    return DK_ERR_ALIGN;
  if (n_rows / kRowsPerBlock >= 0x7fffffff) return DK_ERR_INVALID;
  const dim3 grid(grid_rows(n_rows)), block(kRowThreads);
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, block, 0, stream, x, (const f16*)delta, xout, w, (f16*)y, rstd,
                       (f16*)xq, (f16*)xv, mq, mv, n_rows, (int)d, eps, keep_scale);
  };
  if (d <= 1024) args(rms_fwd_kernel<4>);
  else if (d <= 2048) args(rms_fwd_kernel<8>);
  else args(rms_fwd_kernel<16>);
  DK_CHECK_LAUNCH();
  return 0;
}

extern "C" int dk_rms_bwd(const void* dy, int dy_f32, const float* gscale, const float* x,
                          const void* delta,
                          const float* w, const float* rstd, const float* dres, float* out,
                          const void* lq, const void* lv, void* out16, const uint8_t* mq,
                          const uint8_t* mv, int64_t n_rows, int64_t d, float keep_scale,
                          hipStream_t stream) {
  if (n_rows < 0 || d < 4 || d > 4096 || d % 4) return DK_ERR_INVALID;
  if (n_rows == 0) return 0;
  if (!dy || !gscale || !x || !w || !rstd || !out) return DK_ERR_INVALID;
  if ((lq == nullptr) != (lv == nullptr) || (lq && (!mq || !mv))) return DK_ERR_INVALID;
  if (!dk_aligned(x, 16) || !dk_aligned(w, 16) || !dk_aligned(out, 16) ||
      !dk_aligned(dy, dy_f32 ? 16 : 8) ||
      (dres && !dk_aligned(dres, 16)) || (delta && !dk_aligned(delta, 8)) ||
      (out16 && !dk_aligned(out16, 8)) ||
      (lq && (!dk_aligned(lq, 8) || !dk_aligned(lv, 8) || !dk_aligned(mq, 4) || !dk_aligned(mv, 4))))
    return DK_ERR_ALIGN;
  if (n_rows / kRowsPerBlock >= 0x7fffffff) return DK_ERR_INVALID;
  const dim3 grid(grid_rows(n_rows)), block(kRowThreads);
  auto args = [&](auto kern) {
    hipLaunchKernelGGL(kern, grid, block, 0, stream, dy, gscale, x, (const f16*)delta,
                       w, rstd, dres, out, (const f16*)lq, (const f16*)lv, (f16*)out16, mq, mv,
                       n_rows, (int)d, keep_scale);
  };
  if (dy_f32) {
    if (d <= 1024) args(rms_bwd_kernel<4, true>);
    else if (d <= 2048) args(rms_bwd_kernel<8, true>);
    else args(rms_bwd_kernel<16, true>);
  } else {
    if (d <= 1024) args(rms_bwd_kernel<4, false>);
    else if (d <= 2048) args(rms_bwd_kernel<8, false>);
    else args(rms_bwd_kernel<16, false>);
  }
  DK_CHECK_LAUNCH();
  return 0;
}

static int qkv_shape_ok(int64_t n_rows, int nq, int nkv, int hd) {
  return n_rows >= 0 && nq > 0 && nkv > 0 && hd >= 8 && hd <= 1024 && hd % 8 == 0 &&
         (int64_t)(nq + 2 * nkv) * hd <= (1 << 20) && n_rows / kRowsPerBlock < 0x7fffffff;
}

extern "C" int dk_qkv_epilogue_fwd(void* qkv, const void* lq, const void* lv, const int32_t* pos,
                                   const float* cos_table, const float* sin_table, int64_t n_rows,
                                   float lora_scale, int nq, int nkv, int hd, hipStream_t stream) {
  if (!qkv_shape_ok(n_rows, nq, nkv, hd)) return DK_ERR_INVALID;
  if (n_rows == 0) return 0;
  if (!qkv || !lq || !lv || !pos || !cos_table || !sin_table) return DK_ERR_INVALID;
  if (!dk_aligned(qkv, 8) || !dk_aligned(lq, 8) || !dk_aligned(lv, 8) ||
      !dk_aligned(cos_table, 16) || !dk_aligned(sin_table, 16))
    return DK_ERR_ALIGN;
  hipLaunchKernelGGL(qkv_epilogue_fwd_kernel, dim3(grid_rows(n_rows)), dim3(kRowThreads), 0, stream,
                     (f16*)qkv, (const f16*)lq, (const f16*)lv, pos, cos_table, sin_table, n_rows,
                     lora_scale, nq, nkv, hd);
  DK_CHECK_LAUNCH();
  return 0;
}

extern "C" int dk_qkv_epilogue_bwd(const void* dq, const void* dk, const void* dv, int grads_f32,
                                   const int32_t* pos, const float* cos_table,
                                   const float* sin_table, void* out, int64_t n_rows, int nq,
                                   int nkv, int hd, int gin, hipStream_t stream) {
  if (!qkv_shape_ok(n_rows, nq, nkv, hd) || gin < 1 || gin > 64) return DK_ERR_INVALID;
  if (n_rows == 0) return 0;
  if (!dq || !dk || !dv || !pos || !cos_table || !sin_table || !out) return DK_ERR_INVALID;
  const uintptr_t ga = grads_f32 ? 16 : 8;
  if (!dk_aligned(dq, ga) || !dk_aligned(dk, ga) || !dk_aligned(dv, ga) || !dk_aligned(out, 8) ||
      !dk_aligned(cos_table, 16) || !dk_aligned(sin_table, 16))
    return DK_ERR_ALIGN;
  const dim3 grid(grid_rows(n_rows)), block(kRowThreads);
  if (grads_f32)
    hipLaunchKernelGGL(qkv_epilogue_bwd_kernel<float>, grid, block, 0, stream, (const float*)dq,
                       (const float*)dk, (const float*)dv, pos, cos_table, sin_table, (f16*)out,
                       n_rows, nq, nkv, hd, gin);
  else
    hipLaunchKernelGGL(qkv_epilogue_bwd_kernel<f16>, grid, block, 0, stream, (const f16*)dq,
                       (const f16*)dk, (const f16*)dv, pos, cos_table, sin_table, (f16*)out,
                       n_rows, nq, nkv, hd, gin);
  DK_CHECK_LAUNCH();
  return 0;
}
