// Rank-r LoRA kernels around the NF4 linear (r = 16 in the reference; r in {16, 32, 48, 64}).
//
// Row reductions (one wave per token row, 8 columns per lane per step, 16-byte loads):
//   down:  Xd = fp16(mask ? fp32(x) * ks : 0);  z[m][r] = fp16(sum_k Xd[m][k] A[r][k])
//          (solution/k_norm.py:49-53; solution/fast_qwen.py:943-944)
//   dz:    dz[m][r] = fp16(fp32(fp16(sum_n dY[m][n] B[n][r])) * s)
//          (solution/fast_qwen.py:1370, 1373: mm(gq, B).mul_(s) on an fp16 tensor)
// Column reductions over the token rows, in two deterministic passes (fixed-order partial sums
// per 128-row chunk into a workspace, then one finalize pass):
//   dB[n][r] = fp32(fp16(sum_m dY[m][n] z[m][r])) * s       (solution/fast_qwen.py:1369)
//   dA[r][k] = fp32(fp16(sum_m dz[m][r] Xd[m][k]))           (solution/fast_qwen.py:1371)
// Products of two fp16 values are exact in fp32; only the order of the fp32 sums differs from a
// cuBLAS or CPU GEMM.
#include "dk_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBlock = kThreads / 64;
constexpr int kChunkRows = 256;

__device__ __forceinline__ float wave_sum(float v) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ f16x8 dropout8(const f16x8 x, const uint8_t* mask, float ks) {
  f16x8 out;
  const u32x2 mw = *reinterpret_cast<const u32x2*>(mask);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t keep = (mw[e >> 2] >> (8 * (e & 3))) & 0xffu;
    out[e] = keep ? dk_h(__fmul_rn((float)x[e], ks)) : (f16)0.0f;
  }
  return out;
}

// MODE 0: lora down (weights A [R][cols], optional dropout mask).  MODE 1: dz (weights B
// [cols][R], scale s).
template <int R, int MODE>
__global__ __launch_bounds__(kThreads) void lora_rows_kernel(const f16* __restrict__ in,
                                                             const uint8_t* __restrict__ mask,
                                                             float ks, const f16* __restrict__ wt,
                                                             float scale, f16* __restrict__ out,
                                                             int64_t rows, int64_t cols) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
  if (row >= rows) return;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  const f16* src = in + row * cols;
  for (int64_t c = 8 * lane; c < cols; c += 512) {
    f16x8 x = *reinterpret_cast<const f16x8*>(src + c);
    if (MODE == 0 && mask) x = dropout8(x, mask + row * cols + c, ks);
    if (MODE == 0) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(wt + (int64_t)r * cols + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r] += (float)x[e] * (float)a[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float xe = (float)x[e];
#pragma unroll
        for (int r8 = 0; r8 < R / 8; ++r8) {
          const f16x8 bv = *reinterpret_cast<const f16x8*>(wt + (c + e) * R + 8 * r8);
#pragma unroll
          for (int t = 0; t < 8; ++t) acc[8 * r8 + t] += xe * (float)bv[t];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float s = wave_sum(acc[r]);
    if (lane == r % 64) {
      if (MODE == 0) {
        out[row * R + r] = dk_h(s);
      } else {
        out[row * R + r] = dk_h(__fmul_rn((float)dk_h(s), scale));
      }
    }
  }
}

// Partial column sums over one 256-row chunk: part[chunk][n][r] = sum_m P[m][n] Q[m][r].  A block
// owns 64 columns (one per lane); its 4 waves take every 4th row of the chunk and are summed in a
// fixed order through LDS.  DROP: P is the dropout of x (mask may be null).
template <int R, bool DROP>
__global__ __launch_bounds__(kThreads) void lora_cols_kernel(const f16* __restrict__ P,
                                                             const uint8_t* __restrict__ mask,
                                                             float ks, const f16* __restrict__ Q,
                                                             float* __restrict__ part,
                                                             int64_t rows, int64_t cols) {
  __shared__ float qs[kChunkRows][R];
  __shared__ float red[kRowsPerBlock - 1][64][R + 1];
  const int64_t chunk = blockIdx.y;
  const int64_t r0 = chunk * kChunkRows;
  const int nrows = (int)(rows - r0 < kChunkRows ? rows - r0 : kChunkRows);
  for (int i = threadIdx.x; i < kChunkRows * R; i += kThreads) {
    const int rr = i / R, r = i % R;
    qs[rr][r] = rr < nrows ? (float)Q[(r0 + rr) * R + r] : 0.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t n = (int64_t)blockIdx.x * 64 + lane;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  if (n < cols) {
    // U rows per batch: their loads are all in flight before the first one is used
    constexpr int U = 8;
    for (int rr0 = w; rr0 < nrows; rr0 += kRowsPerBlock * U) {
      float pv[U];
      int rc[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int rr = rr0 + u * kRowsPerBlock;
        rc[u] = rr < nrows ? rr : nrows - 1;
        const int64_t m = r0 + rc[u];
        float v = (float)P[m * cols + n];
        if (DROP && mask) v = mask[m * cols + n] ? (float)dk_h(__fmul_rn(v, ks)) : 0.0f;
        pv[u] = rr < nrows ? v : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] += pv[u] * qs[rc[u]][r];
    }
  }
  if (w > 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) red[w - 1][lane][r] = acc[r];
  }
  __syncthreads();
  if (w == 0 && n < cols) {
    float* dst = part + (chunk * cols + n) * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float s = acc[r];
#pragma unroll
      for (int v = 0; v < kRowsPerBlock - 1; ++v) s += red[v][lane][r];
      dst[r] = s;
    }
  }
}

// out = fp32(fp16(sum over chunks of part[chunk][n][r])) * scale, stored [n][r] or, TRANSPOSE,
// [r][n].
template <bool TRANSPOSE>
__global__ __launch_bounds__(kThreads) void lora_finalize_kernel(const float* __restrict__ part,
                                                                 int64_t n_chunks, int64_t cols,
                                                                 int64_t R, float scale,
                                                                 float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (i >= cols * R) return;
  float s = 0.0f;
  for (int64_t c = 0; c < n_chunks; ++c) s += part[c * cols * R + i];
  const float v = __fmul_rn((float)dk_h(s), scale);
  const int64_t n = i / R, r = i % R;
  if (TRANSPOSE) out[r * cols + n] = v; else out[i] = v;
}

template <int MODE>
int rows_dispatch(int64_t R, dim3 grid, hipStream_t stream, const f16* in, const uint8_t* mask,
                  float ks, const f16* wt, float scale, f16* out, int64_t rows, int64_t cols) {
  switch (R) {
    case 16: hipLaunchKernelGGL((lora_rows_kernel<16, MODE>), grid, dim3(kThreads), 0, stream, in, mask, ks, wt, scale, out, rows, cols); break;
    case 32: hipLaunchKernelGGL((lora_rows_kernel<32, MODE>), grid, dim3(kThreads), 0, stream, in, mask, ks, wt, scale, out, rows, cols); break;
    case 48: hipLaunchKernelGGL((lora_rows_kernel<48, MODE>), grid, dim3(kThreads), 0, stream, in, mask, ks, wt, scale, out, rows, cols); break;
    case 64: hipLaunchKernelGGL((lora_rows_kernel<64, MODE>), grid, dim3(kThreads), 0, stream, in, mask, ks, wt, scale, out, rows, cols); break;
    default: return DK_ERR_INVALID;
  }
  DK_CHECK_LAUNCH();
  return 0;
}

template <bool DROP>
int cols_dispatch(int64_t R, dim3 grid, hipStream_t stream, const f16* P, const uint8_t* mask,
                  float ks, const f16* Q, float* part, int64_t rows, int64_t cols) {
  switch (R) {
    case 16: hipLaunchKernelGGL((lora_cols_kernel<16, DROP>), grid, dim3(kThreads), 0, stream, P, mask, ks, Q, part, rows, cols); break;
    case 32: hipLaunchKernelGGL((lora_cols_kernel<32, DROP>), grid, dim3(kThreads), 0, stream, P, mask, ks, Q, part, rows, cols); break;
    case 48: hipLaunchKernelGGL((lora_cols_kernel<48, DROP>), grid, dim3(kThreads), 0, stream, P, mask, ks, Q, part, rows, cols); break;
    case 64: hipLaunchKernelGGL((lora_cols_kernel<64, DROP>), grid, dim3(kThreads), 0, stream, P, mask, ks, Q, part, rows, cols); break;
    default: return DK_ERR_INVALID;
  }
  DK_CHECK_LAUNCH();
  return 0;
}

bool rank_ok(int64_t r) { return r >= 16 && r <= 64 && r % 16 == 0; }

}  // namespace

extern "C" int dk_lora_down(const void* x, const uint8_t* mask, float keep_scale, const void* a,
                            void* z, int64_t m, int64_t k, int64_t rank, hipStream_t stream) {
  if (m < 0 || k <= 0 || k % 8 || !rank_ok(rank) || !x || !a || !z) return DK_ERR_INVALID;
  if (!dk_aligned(x, 16) || !dk_aligned(a, 16) || (mask && !dk_aligned(mask, 8))) return DK_ERR_ALIGN;
  if (m == 0) return 0;
  dim3 grid((unsigned)((m + kRowsPerBlock - 1) / kRowsPerBlock));
  return rows_dispatch<0>(rank, grid, stream, (const f16*)x, mask, mask ? keep_scale : 1.0f,
                          (const f16*)a, 1.0f, (f16*)z, m, k);
}

extern "C" int64_t dk_lora_grads_workspace(int64_t m, int64_t n_out, int64_t k, int64_t rank) {
  if (m <= 0) return 0;
  const int64_t chunks = (m + kChunkRows - 1) / kChunkRows;
  const int64_t cols = n_out > k ? n_out : k;
  return chunks * cols * rank * (int64_t)sizeof(float);
}

extern "C" int dk_lora_grads(const void* dy, const void* z, const void* x, const uint8_t* mask,
                             float keep_scale, const void* lora_b, float lora_scale, int64_t m,
                             int64_t n_out, int64_t k, int64_t rank, float* da, float* db,
                             void* dz, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (m < 0 || n_out <= 0 || k <= 0 || n_out % 8 || k % 8 || !rank_ok(rank)) return DK_ERR_INVALID;
  if (!dy || !z || !x || !lora_b || !da || !db || !dz) return DK_ERR_INVALID;
  if (!dk_aligned(dy, 16) || !dk_aligned(x, 16) || !dk_aligned(lora_b, 16) ||
      (mask && !dk_aligned(mask, 8)))
    return DK_ERR_ALIGN;
  if (m == 0) return 0;
  if (!ws || ws_bytes < dk_lora_grads_workspace(m, n_out, k, rank)) return DK_ERR_WORKSPACE;
  const float ks = mask ? keep_scale : 1.0f;
  const int64_t chunks = (m + kChunkRows - 1) / kChunkRows;
  float* part = (float*)ws;
  // dz = fp16(fp16(dY B) * s)
  int e = rows_dispatch<1>(rank, dim3((unsigned)((m + kRowsPerBlock - 1) / kRowsPerBlock)), stream,
                           (const f16*)dy, nullptr, 1.0f, (const f16*)lora_b, lora_scale,
                           (f16*)dz, m, n_out);
  if (e) return e;
  // dB = fp32(fp16(dY^T z)) * s
  e = cols_dispatch<false>(rank, dim3((unsigned)((n_out + 63) / 64), (unsigned)chunks),
                           stream, (const f16*)dy, nullptr, 1.0f, (const f16*)z, part, m, n_out);
  if (e) return e;
  hipLaunchKernelGGL(lora_finalize_kernel<false>, dim3((unsigned)((n_out * rank + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, part, chunks, n_out, rank, lora_scale, db);
  DK_CHECK_LAUNCH();
  // dA = fp32(fp16(dz^T Xd))
  e = cols_dispatch<true>(rank, dim3((unsigned)((k + 63) / 64), (unsigned)chunks),
                          stream, (const f16*)x, mask, ks, (const f16*)dz, part, m, k);
  if (e) return e;
  hipLaunchKernelGGL(lora_finalize_kernel<true>, dim3((unsigned)((k * rank + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, part, chunks, k, rank, 1.0f, da);
  DK_CHECK_LAUNCH();
  return 0;
}
