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

__device__ __forceinline__ f32x4 to_f4(const f16x4 h) {
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
  const int kn = (d + 255) / 256;   // chunks holding any of the row (uniform)
  // every load of the row first, at clamped addresses (a lane past the row reads element 0 and
  // its values are not used), then the arithmetic: a load consumed right away would make the
  // compiler wait for it before the next chunk's loads go out, one memory latency per chunk
  // Straight-line loads (a load under a branch, or converted at once, makes the compiler wait for
  // it there): every chunk up to KMAX, and the optional inputs from x when absent (read, unused).
  const f16* dsrc = delta ? delta : reinterpret_cast<const f16*>(x);
  const uint8_t* qsrc = xq ? mq : reinterpret_cast<const uint8_t*>(x);
  const uint8_t* vsrc = xq ? mv : reinterpret_cast<const uint8_t*>(x);
  f32x4 h[KMAX], wv[KMAX];
  f16x4 dl[KMAX];
  uint32_t kq[KMAX], kv[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int e = 256 * k + 4 * lane, ec = e < d ? e : 0;
    h[k] = *reinterpret_cast<const f32x4*>(x + off + ec);
    wv[k] = *reinterpret_cast<const f32x4*>(w + ec);
    kq[k] = load_mask4(qsrc + off + ec);
    kv[k] = load_mask4(vsrc + off + ec);
    dl[k] = *reinterpret_cast<const f16x4*>(dsrc + off + ec);
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    if (k >= kn) continue;
    const int e = 256 * k + 4 * lane;
    if (delta) {
      const f32x4 d4 = to_f4(dl[k]);
#pragma unroll
      for (int i = 0; i < 4; ++i) h[k][i] = __fadd_rn(h[k][i], d4[i]);
    }
    float sk = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) sk = __fadd_rn(sk, __fmul_rn(h[k][i], h[k][i]));
    // (the per-chunk partial then the running sum: the same order as summing element by element
    // would not be; both are a lane-order sum of this lane's squares)
    ss = e < d ? __fadd_rn(ss, sk) : ss;
    if (xout && e < d) *reinterpret_cast<f32x4*>(xout + off + e) = h[k];
  }
  const float ms = __fmul_rn(wave_sum(ss), 1.0f / (float)d);
  const float r = rsqrtf(__fadd_rn(ms, eps));
  if (lane == 0) rstd[row] = r;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int e = 256 * k + 4 * lane;
    if (k >= kn || e >= d) continue;
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
  const int kn = (d + 255) / 256;   // chunks holding any of the row (uniform)
  // every load of the row first, at clamped addresses (lanes past the row read element 0 and
  // their values are not used), then the arithmetic
  // fp16 operands are kept as loaded and converted after the loads (a conversion here would wait
  // for its load)
  // straight-line loads: every chunk up to KMAX, and the optional inputs from x when absent
  // (read, unused); dres before the reduction, since out may alias it
  const f16* x16 = reinterpret_cast<const f16*>(x);
  const uint8_t* x8 = reinterpret_cast<const uint8_t*>(x);
  const f16* lqs = lq ? lq : x16;
  const f16* lvs = lq ? lv : x16;
  const uint8_t* mqs = lq ? mq : x8;
  const uint8_t* mvs = lq ? mv : x8;
  const f16* dls = delta ? delta : x16;
  const float* rvs = dres ? dres : x;
  f32x4 dy32[KMAX], xv[KMAX], wv[KMAX], rv[KMAX];
  f16x4 dy16[KMAX], a[KMAX], b[KMAX], dl[KMAX];
  uint32_t kq[KMAX], kv[KMAX];
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int e = 256 * k + 4 * lane, ec = e < d ? e : 0;
    if (DY32) dy32[k] = *reinterpret_cast<const f32x4*>(static_cast<const float*>(dyp) + off + ec);
    else dy16[k] = *reinterpret_cast<const f16x4*>(static_cast<const f16*>(dyp) + off + ec);
    kq[k] = load_mask4(mqs + off + ec);
    kv[k] = load_mask4(mvs + off + ec);
    a[k] = *reinterpret_cast<const f16x4*>(lqs + off + ec);
    b[k] = *reinterpret_cast<const f16x4*>(lvs + off + ec);
    xv[k] = *reinterpret_cast<const f32x4*>(x + off + ec);
    dl[k] = *reinterpret_cast<const f16x4*>(dls + off + ec);
    wv[k] = *reinterpret_cast<const f32x4*>(w + ec);
    rv[k] = *reinterpret_cast<const f32x4*>(rvs + off + ec);
  }
  f32x4 g[KMAX], xh[KMAX];
  float cs = 0.0f;
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    if (k >= kn) continue;
    const int e = 256 * k + 4 * lane;
    f32x4 dyk = DY32 ? dy32[k] : to_f4(dy16[k]);
#pragma unroll
    for (int i = 0; i < 4; ++i) dyk[i] = __fmul_rn(dyk[i], gs);
    if (lq) {
      const f32x4 ak = to_f4(a[k]), bk = to_f4(b[k]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        dyk[i] = __fadd_rn(dyk[i], kept(kq[k], i) ? __fmul_rn(ak[i], keep_scale) : 0.0f);
        dyk[i] = __fadd_rn(dyk[i], kept(kv[k], i) ? __fmul_rn(bk[i], keep_scale) : 0.0f);
      }
    }
    if (delta) {
      const f32x4 d4 = to_f4(dl[k]);
#pragma unroll
      for (int i = 0; i < 4; ++i) xv[k][i] = __fadd_rn(xv[k][i], d4[i]);
    }
    float ck = cs;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      xh[k][i] = __fmul_rn(xv[k][i], r);
      g[k][i] = __fmul_rn(dyk[i], wv[k][i]);
      ck = __fadd_rn(ck, __fmul_rn(g[k][i], xh[k][i]));
    }
    cs = e < d ? ck : cs;
  }
  const float c = __fmul_rn(wave_sum(cs), 1.0f / (float)d);
#pragma unroll
  for (int k = 0; k < KMAX; ++k) {
    const int e = 256 * k + 4 * lane;
    if (k >= kn || e >= d) continue;
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
  // (loads at clamped tasks, straight-line, fp16 converted after: a load under a branch or used
  // at once makes the compiler wait for it there)
  const int tasks = (nq + nkv) * quads;
  for (int t0 = 0; t0 < tasks; t0 += 64 * kBatch) {
    f16x4 x1h[kBatch], x2h[kBatch], ah[kBatch], bh[kBatch];
    f32x4 c[kBatch], s[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t0u = t0 + 64 * u + lane, t = t0u < tasks ? t0u : tasks - 1;
      const int head = t / quads, j = 4 * (t % quads);
      const f16* h1 = base + head * hd + j;
      x1h[u] = *reinterpret_cast<const f16x4*>(h1);
      x2h[u] = *reinterpret_cast<const f16x4*>(h1 + half);
      c[u] = *reinterpret_cast<const f32x4*>(cr + j);
      s[u] = *reinterpret_cast<const f32x4*>(sr + j);
      const int hq = head < nq ? head : nq - 1;   // key heads: read, unused
      ah[u] = *reinterpret_cast<const f16x4*>(lqr + hq * hd + j);
      bh[u] = *reinterpret_cast<const f16x4*>(lqr + hq * hd + j + half);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= tasks) continue;
      const int head = t / quads, j = 4 * (t % quads);
      f32x4 x1 = to_f4(x1h[u]), x2 = to_f4(x2h[u]);
      if (head < nq) {
        const f32x4 a = to_f4(ah[u]), b = to_f4(bh[u]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x1[i] = __fadd_rn(x1[i], __fmul_rn(a[i], scale));
          x2[i] = __fadd_rn(x2[i], __fmul_rn(b[i], scale));
        }
      }
      f32x4 o1, o2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o1[i] = __fsub_rn(__fmul_rn(x1[i], c[u][i]), __fmul_rn(x2[i], s[u][i]));
        o2[i] = __fadd_rn(__fmul_rn(x2[i], c[u][i]), __fmul_rn(x1[i], s[u][i]));
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
    f16x4 vh[kBatch], ah[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t0u = t0 + 64 * u + lane, t = t0u < vtasks ? t0u : vtasks - 1;
      vh[u] = *reinterpret_cast<const f16x4*>(vb + 4 * t);
      ah[u] = *reinterpret_cast<const f16x4*>(lvr + 4 * t);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= vtasks) continue;
      f32x4 v = to_f4(vh[u]);
      const f32x4 a = to_f4(ah[u]);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = __fadd_rn(v[i], __fmul_rn(a[i], scale));
      store_h4(vb + 4 * t, v);
    }
  }
}

// Four elements of a gradient that arrives as fp32 or fp16: loaded raw, converted at use (a
// conversion right after the load would make the compiler wait for that load there).
template <typename T>
using Raw4 = std::conditional_t<sizeof(T) == 4, f32x4, f16x4>;

template <typename T>
__device__ __forceinline__ Raw4<T> raw4(const T* p) {
  return *reinterpret_cast<const Raw4<T>*>(p);
}

__device__ __forceinline__ f32x4 cvt4(f32x4 v) { return v; }
__device__ __forceinline__ f32x4 cvt4(f16x4 v) { return to_f4(v); }

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
    Raw4<T> d1[kBatch], d2[kBatch];
    f32x4 c[kBatch], s[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {   // clamped tasks: straight-line loads
      const int t0u = t0 + 64 * u + lane, t = t0u < qtasks ? t0u : qtasks - 1;
      const int head = t / quads, j = 4 * (t % quads);
      d1[u] = raw4(dqr + head * hd + j);
      d2[u] = raw4(dqr + head * hd + j + half);
      c[u] = *reinterpret_cast<const f32x4*>(cr + j);
      s[u] = *reinterpret_cast<const f32x4*>(sr + j);
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int t = t0 + 64 * u + lane;
      if (t >= qtasks) continue;
      const int head = t / quads, j = 4 * (t % quads);
      const f32x4 a = cvt4(d1[u]), b = cvt4(d2[u]);
      f32x4 o1, o2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        o1[i] = __fadd_rn(__fmul_rn(a[i], c[u][i]), __fmul_rn(b[i], s[u][i]));
        o2[i] = __fsub_rn(__fmul_rn(b[i], c[u][i]), __fmul_rn(a[i], s[u][i]));
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
      Raw4<T> pa[kGinBatch], pb[kGinBatch];
#pragma unroll
      for (int u = 0; u < kGinBatch; ++u) {   // partials past gin: the last one read, unused
        const int g = g0 + u < gin ? g0 + u : gin - 1;
        const T* part = dkr + (int64_t)(hk * gin + g) * hd + j;
        pa[u] = raw4(part);
        pb[u] = raw4(part + half);
      }
#pragma unroll
      for (int u = 0; u < kGinBatch; ++u) {
        if (g0 + u >= gin) continue;
        const f32x4 a = cvt4(pa[u]), b = cvt4(pb[u]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          d1[i] = __fadd_rn(d1[i], a[i]);
          d2[i] = __fadd_rn(d2[i], b[i]);
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
      Raw4<T> pa[kGinBatch];
#pragma unroll
      for (int u = 0; u < kGinBatch; ++u) {
        const int g = g0 + u < gin ? g0 + u : gin - 1;
        pa[u] = raw4(dvr + (int64_t)(hk * gin + g) * hd + e);
      }
#pragma unroll
      for (int u = 0; u < kGinBatch; ++u) {
        if (g0 + u >= gin) continue;
        const f32x4 a = cvt4(pa[u]);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = __fadd_rn(acc[i], a[i]);
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
  // (the chunk count sets the registers a row's loads hold: at most 1536 columns, Qwen2.5-1.5B's
  // hidden size, keeps the backward at two waves per SIMD)
  if (d <= 1024) args(rms_fwd_kernel<4>);
  else if (d <= 1536) args(rms_fwd_kernel<6>);
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
    else if (d <= 1536) args(rms_bwd_kernel<6, true>);
    else if (d <= 2048) args(rms_bwd_kernel<8, true>);
    else args(rms_bwd_kernel<16, true>);
  } else {
    if (d <= 1024) args(rms_bwd_kernel<4, false>);
    else if (d <= 1536) args(rms_bwd_kernel<6, false>);
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
