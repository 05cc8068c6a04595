// Rank-r LoRA kernels around the NF4 linear (r = 16 in the reference; r in {16, 32, 48, 64}).
//
// Row reductions (MFMA v_mfma_f32_16x16x32_f16; a workgroup owns 16 token rows and its 4 waves
// split K, summed in a fixed order through LDS):
//   down:  Xd = fp16(mask ? fp32(x) * ks : 0);  z[m][r] = fp16(sum_k Xd[m][k] A[r][k])
//          (solution/k_norm.py:49-53; solution/fast_qwen.py:943-944)
//   dz:    dz[m][r] = fp16(fp32(fp16(sum_n dY[m][n] B[n][r])) * s)
//          (solution/fast_qwen.py:1370, 1373: mm(gq, B).mul_(s) on an fp16 tensor)
//          B is staged transposed in LDS so its MFMA operand is K-contiguous.
// Column reductions over the token rows, in two deterministic passes (fixed-order partial sums
// per 64-row chunk into a workspace, then one finalize pass):
//   dB[n][r] = fp32(fp16(sum_m dY[m][n] z[m][r])) * s       (solution/fast_qwen.py:1369)
//   dA[r][k] = fp32(fp16(sum_m dz[m][r] Xd[m][k]))           (solution/fast_qwen.py:1371)
// Products of two fp16 values are exact in fp32; only the order of the fp32 sums differs from a
// cuBLAS or CPU GEMM.
#include "dk_common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kRowTile = 16;     // rows per workgroup of the row reductions
constexpr int kChunkRows = 64;   // rows per partial sum of the column reductions
constexpr int kColsPerBlock = 128;

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

// MODE 0 (down): out[m][r] = fp16(sum_k Xd[m][k] W[r][k]), W = A [R][cols].
// MODE 1 (dz):   out[m][r] = fp16(fp16(sum_k in[m][k] W[k][r]) * scale), W = B [cols][R], staged
//                transposed in LDS.
// 16x16x32 MFMA operand layout: lane l holds row/column l % 16 and k = 8 * (l / 16) + [0, 8);
// the result register v of lane l is row 4 * (l / 16) + v, column l % 16.
template <int R, int MODE>
__global__ __launch_bounds__(kThreads) void lora_rows_kernel(const f16* __restrict__ in,
                                                             int64_t ld,
                                                             const uint8_t* __restrict__ mask,
                                                             float ks, const f16* __restrict__ wt,
                                                             float scale, f16* __restrict__ out,
                                                             int64_t rows, int64_t cols) {
  constexpr int RB = R / 16;
  constexpr int KC = 1024;  // columns of B^T staged per pass (MODE 1)
  __shared__ float red[kWaves * 16 * R];
  __shared__ __attribute__((aligned(16))) f16 wT[MODE == 1 ? R * (KC + 8) : 8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * kRowTile;
  const int lr = lane & 15, lk = 8 * (lane >> 4);
  const int64_t m = row0 + lr < rows ? row0 + lr : rows - 1;   // clamped: its sums are not stored
  f32x4 acc[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (MODE == 0) {
    for (int64_t s = w; s < cols / 32; s += kWaves) {
      const int64_t k = s * 32 + lk;
      f16x8 a = *reinterpret_cast<const f16x8*>(in + m * ld + k);
      if (mask) a = dropout8(a, mask + m * cols + k, ks);
#pragma unroll
      for (int b = 0; b < RB; ++b) {
        const f16x8 bw = *reinterpret_cast<const f16x8*>(wt + (int64_t)(16 * b + lr) * cols + k);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw, acc[b], 0, 0, 0);
      }
    }
  } else {
    for (int64_t c0 = 0; c0 < cols; c0 += KC) {
      const int kc = (int)(cols - c0 < KC ? cols - c0 : KC);
      __syncthreads();  // the previous pass has finished reading wT
      // B^T columns [c0, c0 + kc) into LDS: 8 consecutive r of one k per thread, scattered
      for (int i = tid; i < kc * (R / 8); i += kThreads) {
        const int kk = i / (R / 8), r8 = (i % (R / 8)) * 8;
        const f16x8 v = *reinterpret_cast<const f16x8*>(wt + (c0 + kk) * R + r8);
#pragma unroll
        for (int e = 0; e < 8; ++e) wT[(r8 + e) * (KC + 8) + kk] = v[e];
      }
      __syncthreads();
      for (int s = w; s < kc / 32; s += kWaves) {
        const f16x8 a = *reinterpret_cast<const f16x8*>(in + m * ld + c0 + s * 32 + lk);
#pragma unroll
        for (int b = 0; b < RB; ++b) {
          const f16x8 bw = *reinterpret_cast<const f16x8*>(wT + (16 * b + lr) * (KC + 8) + s * 32 + lk);
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw, acc[b], 0, 0, 0);
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < RB; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[(w * 16 + 4 * (lane >> 4) + v) * R + 16 * b + lr] = acc[b][v];
  __syncthreads();
  for (int i = tid; i < 16 * R; i += kThreads) {
    const int rr = i / R, r = i % R;
    if (row0 + rr >= rows) continue;
    float sum = 0.0f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) sum += red[(ww * 16 + rr) * R + r];
    out[(row0 + rr) * R + r] = MODE == 0 ? dk_h(sum) : dk_h(__fmul_rn((float)dk_h(sum), scale));
  }
}

// Partial column sums over one 64-row chunk: part[chunk][n][r] = sum_m P[m][n] Q[m][r].  A block
// owns 128 columns (two per lane); its 4 waves take 16 rows each, all 16 loads in flight before
// the first use, and are summed in a fixed order through LDS.  DROP: P is the dropout of x (mask
// may be null).
template <int R, bool DROP>
__global__ __launch_bounds__(kThreads) void lora_cols_kernel(const f16* __restrict__ P, int64_t ld,
                                                             const uint8_t* __restrict__ mask,
                                                             float ks, const f16* __restrict__ Q,
                                                             float* __restrict__ part,
                                                             int64_t rows, int64_t cols) {
  constexpr int RW = kChunkRows / kWaves;  // rows per wave
  __shared__ __attribute__((aligned(16))) float qs[kChunkRows][R];
  __shared__ float red[kWaves - 1][64][2 * R + 1];
  const int64_t chunk = blockIdx.y;
  const int64_t r0 = chunk * kChunkRows;
  const int nrows = (int)(rows - r0 < kChunkRows ? rows - r0 : kChunkRows);
  for (int i = threadIdx.x; i < kChunkRows * R; i += kThreads) {
    const int rr = i / R, r = i % R;
    qs[rr][r] = rr < nrows ? (float)Q[(r0 + rr) * R + r] : 0.0f;
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t n = (int64_t)blockIdx.x * kColsPerBlock + 2 * lane;
  const bool live = n < cols;
  const int64_t nc = live ? n : 0;
  float p0[RW], p1[RW];
#pragma unroll
  for (int u = 0; u < RW; ++u) {
    const int rr = w * RW + u;
    const int rc = rr < nrows ? rr : nrows - 1;
    const int64_t m = r0 + rc;
    const f16x2 pv = *reinterpret_cast<const f16x2*>(P + m * ld + nc);
    float a = (float)pv[0], b = (float)pv[1];
    if (DROP && mask) {
      const uint32_t mk = *reinterpret_cast<const uint16_t*>(mask + m * cols + nc);
      a = (mk & 0xffu) ? (float)dk_h(__fmul_rn(a, ks)) : 0.0f;
      b = (mk >> 8) ? (float)dk_h(__fmul_rn(b, ks)) : 0.0f;
    }
    p0[u] = rr < nrows ? a : 0.0f;
    p1[u] = rr < nrows ? b : 0.0f;
  }
  float acc0[R], acc1[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc0[r] = acc1[r] = 0.0f;
#pragma unroll
  for (int u = 0; u < RW; ++u) {
    const float* q = qs[w * RW + u];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      acc0[r] += p0[u] * q[r];
      acc1[r] += p1[u] * q[r];
    }
  }
  if (w > 0) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      red[w - 1][lane][r] = acc0[r];
      red[w - 1][lane][R + r] = acc1[r];
    }
  }
  __syncthreads();
  if (w == 0 && live) {
    float* dst = part + (chunk * cols + n) * R;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      float s0 = acc0[r], s1 = acc1[r];
#pragma unroll
      for (int v = 0; v < kWaves - 1; ++v) {
        s0 += red[v][lane][r];
        s1 += red[v][lane][R + r];
      }
      dst[r] = s0;
      dst[R + r] = s1;
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
  // 8 loads in flight at a time, added in chunk order
  float s = 0.0f;
  int64_t c = 0;
  for (; c + 8 <= n_chunks; c += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part[(c + u) * cols * R + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; c < n_chunks; ++c) s += part[c * cols * R + i];
  const float v = __fmul_rn((float)dk_h(s), scale);
  const int64_t n = i / R, r = i % R;
  if (TRANSPOSE) out[r * cols + n] = v; else out[i] = v;
}

template <int MODE>
int rows_dispatch(int64_t R, hipStream_t stream, const f16* in, int64_t ld, const uint8_t* mask,
                  float ks, const f16* wt, float scale, f16* out, int64_t rows, int64_t cols) {
  const dim3 grid((unsigned)((rows + kRowTile - 1) / kRowTile));
  switch (R) {
    case 16: hipLaunchKernelGGL((lora_rows_kernel<16, MODE>), grid, dim3(kThreads), 0, stream, in, ld, mask, ks, wt, scale, out, rows, cols); break;
    case 32: hipLaunchKernelGGL((lora_rows_kernel<32, MODE>), grid, dim3(kThreads), 0, stream, in, ld, mask, ks, wt, scale, out, rows, cols); break;
    case 48: hipLaunchKernelGGL((lora_rows_kernel<48, MODE>), grid, dim3(kThreads), 0, stream, in, ld, mask, ks, wt, scale, out, rows, cols); break;
    case 64: hipLaunchKernelGGL((lora_rows_kernel<64, MODE>), grid, dim3(kThreads), 0, stream, in, ld, mask, ks, wt, scale, out, rows, cols); break;
    default: return DK_ERR_INVALID;
  }
  DK_CHECK_LAUNCH();
  return 0;
}

template <bool DROP>
int cols_dispatch(int64_t R, hipStream_t stream, const f16* P, int64_t ld, const uint8_t* mask,
                  float ks, const f16* Q, float* part, int64_t rows, int64_t cols) {
  const dim3 grid((unsigned)((cols + kColsPerBlock - 1) / kColsPerBlock),
                  (unsigned)((rows + kChunkRows - 1) / kChunkRows));
  switch (R) {
    case 16: hipLaunchKernelGGL((lora_cols_kernel<16, DROP>), grid, dim3(kThreads), 0, stream, P, ld, mask, ks, Q, part, rows, cols); break;
    case 32: hipLaunchKernelGGL((lora_cols_kernel<32, DROP>), grid, dim3(kThreads), 0, stream, P, ld, mask, ks, Q, part, rows, cols); break;
    case 48: hipLaunchKernelGGL((lora_cols_kernel<48, DROP>), grid, dim3(kThreads), 0, stream, P, ld, mask, ks, Q, part, rows, cols); break;
    case 64: hipLaunchKernelGGL((lora_cols_kernel<64, DROP>), grid, dim3(kThreads), 0, stream, P, ld, mask, ks, Q, part, rows, cols); break;
    default: return DK_ERR_INVALID;
  }
  DK_CHECK_LAUNCH();
  return 0;
}

bool rank_ok(int64_t r) { return r >= 16 && r <= 64 && r % 16 == 0; }

}  // namespace

extern "C" int dk_lora_down(const void* x, const uint8_t* mask, float keep_scale, const void* a,
                            void* z, int64_t m, int64_t k, int64_t rank, hipStream_t stream) {
  if (m < 0 || k <= 0 || k % 32 || !rank_ok(rank) || !x || !a || !z) return DK_ERR_INVALID;
  if (!dk_aligned(x, 16) || !dk_aligned(a, 16) || (mask && !dk_aligned(mask, 8))) return DK_ERR_ALIGN;
  if (m == 0) return 0;
  return rows_dispatch<0>(rank, stream, (const f16*)x, k, mask, mask ? keep_scale : 1.0f,
                          (const f16*)a, 1.0f, (f16*)z, m, k);
}

extern "C" int64_t dk_lora_grads_workspace(int64_t m, int64_t n_out, int64_t k, int64_t rank) {
  if (m <= 0) return 0;
  const int64_t chunks = (m + kChunkRows - 1) / kChunkRows;
  const int64_t cols = n_out > k ? n_out : k;
  return chunks * cols * rank * (int64_t)sizeof(float);
}

extern "C" int dk_lora_grads(const void* dy, int64_t lddy, const void* z, const void* x,
                             const uint8_t* mask,
                             float keep_scale, const void* lora_b, float lora_scale, int64_t m,
                             int64_t n_out, int64_t k, int64_t rank, float* da, float* db,
                             void* dz, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (m < 0 || n_out <= 0 || k <= 0 || n_out % 32 || k % 32 || !rank_ok(rank)) return DK_ERR_INVALID;
  if (!dy || !z || !x || !lora_b || !da || !db || !dz || lddy < n_out) return DK_ERR_INVALID;
  if (!dk_aligned(dy, 16) || lddy % 8 || !dk_aligned(x, 16) || !dk_aligned(lora_b, 16) ||
      (mask && !dk_aligned(mask, 8)))
    return DK_ERR_ALIGN;
  if (m == 0) return 0;
  if (!ws || ws_bytes < dk_lora_grads_workspace(m, n_out, k, rank)) return DK_ERR_WORKSPACE;
  const float ks = mask ? keep_scale : 1.0f;
  const int64_t chunks = (m + kChunkRows - 1) / kChunkRows;
  float* part = (float*)ws;
  // dz = fp16(fp16(dY B) * s)
  int e = rows_dispatch<1>(rank, stream, (const f16*)dy, lddy, nullptr, 1.0f, (const f16*)lora_b,
                           lora_scale, (f16*)dz, m, n_out);
  if (e) return e;
  // dB = fp32(fp16(dY^T z)) * s
  e = cols_dispatch<false>(rank, stream, (const f16*)dy, lddy, nullptr, 1.0f, (const f16*)z, part, m,
                           n_out);
  if (e) return e;
  hipLaunchKernelGGL(lora_finalize_kernel<false>, dim3((unsigned)((n_out * rank + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, part, chunks, n_out, rank, lora_scale, db);
  DK_CHECK_LAUNCH();
  // dA = fp32(fp16(dz^T Xd))
  e = cols_dispatch<true>(rank, stream, (const f16*)x, k, mask, ks, (const f16*)dz, part, m, k);
  if (e) return e;
  hipLaunchKernelGGL(lora_finalize_kernel<true>, dim3((unsigned)((k * rank + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, part, chunks, k, rank, 1.0f, da);
  DK_CHECK_LAUNCH();
  return 0;
}
