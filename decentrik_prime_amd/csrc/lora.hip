// Rank-r LoRA kernels around the NF4 linear (r = 16 in the reference; r in {16, 32, 48, 64}).
//
// Row reductions (MFMA v_mfma_f32_16x16x32_f16; a workgroup owns 16 token rows and its 8 waves
// split K, summed in a fixed order through LDS):
//   down:  Xd = fp16(mask ? fp32(x) * ks : 0);  z[m][r] = fp16(sum_k Xd[m][k] A[r][k])
//          (solution/k_norm.py:49-53; solution/fast_qwen.py:943-944)
//   dz:    dz[m][r] = fp16(fp32(fp16(sum_n dY[m][n] B[n][r])) * s)
//          (solution/fast_qwen.py:1370, 1373: mm(gq, B).mul_(s) on an fp16 tensor)
//          B is staged in LDS as stored and read K-contiguous with transposing LDS reads.
// Column reductions over all token rows in one deterministic pass (a workgroup per 32 columns,
// MFMA on LDS-staged 32-row chunks, the waves' sums added in a fixed order):
//   dB[n][r] = fp32(fp16(sum_m dY[m][n] z[m][r])) * s       (solution/fast_qwen.py:1369)
//   dA[r][k] = fp32(fp16(sum_m dz[m][r] Xd[m][k]))           (solution/fast_qwen.py:1371)
// Products of two fp16 values are exact in fp32; only the order of the fp32 sums differs from a
// cuBLAS or CPU GEMM.
#include "dk_common.h"

namespace {

constexpr int kRowTile = 16;     // rows per workgroup of the row reductions
constexpr int kRowThreads = 512; // 8 waves split K in the row reductions
constexpr int kMaxJobs = 2;      // LoRA terms per launch (q and v of the fused QKV projection)

__device__ __forceinline__ f16x8 dropout8(const f16x8 x, const u32x2 mw, float ks) {
  f16x8 out;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t keep = (mw[e >> 2] >> (8 * (e & 3))) & 0xffu;
    const f16 kept = dk_h(__fmul_rn((float)x[e], ks));   // unconditional, then selected
    out[e] = keep ? kept : (f16)0.0f;
  }
  return out;
}

// MODE 0 (down): out[m][r] = fp16(sum_k Xd[m][k] W[r][k]), W = A [R][cols].
// MODE 1 (dz):   out[m][r] = fp16(fp16(sum_k in[m][k] W[k][r]) * scale), W = B [cols][R], staged
//                row-major in LDS and read k-contiguous with ds_read_b64_tr_b16 (see
//                lora_colsum_kernel for the lane layout).
// 16x16x32 MFMA operand layout: lane l holds row/column l % 16 and k = 8 * (l / 16) + [0, 8);
// the result register v of lane l is row 4 * (l / 16) + v, column l % 16.  The 8 waves split K
// and issue the loads of kBatch steps before their MFMAs; their sums are added in a fixed order.
// Up to kMaxJobs independent problems over the same rows run in one launch (the q and v LoRA
// terms of the fused QKV projection); workgroup b serves job b / ceil(rows / kRowTile).
struct RowsJob {
  const f16* in;
  int64_t ld;
  const uint8_t* mask;
  float ks;
  const f16* wt;
  float scale;
  f16* out;
  int64_t cols;
};
struct RowsJobs {
  RowsJob j[kMaxJobs];
};

template <int R, int MODE, bool MASKED>
__global__ __launch_bounds__(kRowThreads) void lora_rows_kernel(RowsJobs jobs, int64_t rows) {
  const int64_t per_job = (rows + kRowTile - 1) / kRowTile;
  const RowsJob& J = jobs.j[blockIdx.x / per_job];
  const f16* __restrict__ in = J.in;
  const int64_t ld = J.ld;
  const uint8_t* __restrict__ mask = J.mask;
  const float ks = J.ks;
  const f16* __restrict__ wt = J.wt;
  const float scale = J.scale;
  f16* __restrict__ out = J.out;
  const int64_t cols = J.cols;
  constexpr int RB = R / 16;
  constexpr int NW = kRowThreads / 64;
  constexpr int kBatch = 6;      // MODE 0: K steps per wave whose loads are in flight together
  constexpr int KC = R == 16 ? 1536 : 768;   // rows of B staged per pass (MODE 1)
  constexpr int KU = KC / 32 / NW;           // MODE 1: dY steps per wave per pass
  constexpr int BI = KC * (R / 8) / kRowThreads;   // MODE 1: 16-byte B pieces per thread per pass
  constexpr int BLD = R + 8;     // halves per staged B row
  static_assert(KU * 32 * NW == KC && BI * kRowThreads == KC * (R / 8), "MODE 1 pass shape");
  __shared__ float red[NW * 16 * R];
  __shared__ __attribute__((aligned(16))) f16 Bs[MODE == 1 ? KC * BLD : 8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t row0 = (int64_t)(blockIdx.x % per_job) * kRowTile;
  const int lr = lane & 15, lk = 8 * (lane >> 4);
  const int64_t m = row0 + lr < rows ? row0 + lr : rows - 1;   // clamped: its sums are not stored
  const int trow = 8 * (lane >> 4) + ((lane & 15) >> 2), tcol = 4 * (lane & 3);
  f32x4 acc[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (MODE == 0) {
    const int64_t steps = cols / 32;
    for (int64_t s0 = w; s0 < steps; s0 += NW * kBatch) {
      f16x8 a[kBatch], bw[kBatch][RB];
      u32x2 mw[kBatch];
      // every load of the batch first (x, keep-mask bytes, A), then the dropout and the MFMAs
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int64_t s = s0 + (int64_t)u * NW;
        const int64_t k = (s < steps ? s : steps - 1) * 32 + lk;   // clamped; not accumulated
        a[u] = *reinterpret_cast<const f16x8*>(in + m * ld + k);
        if (MASKED) mw[u] = *reinterpret_cast<const u32x2*>(mask + m * cols + k);
#pragma unroll
        for (int b = 0; b < RB; ++b)
          bw[u][b] = *reinterpret_cast<const f16x8*>(wt + (int64_t)(16 * b + lr) * cols + k);
      }
      __builtin_amdgcn_sched_barrier(0);   // the batch's loads stay ahead of their first use
      // straight-line (a step past the end multiplies zeros), so no load is sunk below a branch
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (MASKED) a[u] = dropout8(a[u], mw[u], ks);
        const bool valid = s0 + (int64_t)u * NW < steps;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[u][e] = valid ? a[u][e] : (f16)0.0f;
#pragma unroll
        for (int b = 0; b < RB; ++b)
          acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], bw[u][b], acc[b], 0, 0, 0);
      }
    }
  } else {
    // per pass: this wave's dY operands (steps w, w + NW, ...) and this thread's pieces of B are
    // all loaded before the first is used, then B goes to LDS behind one barrier
    for (int64_t c0 = 0; c0 < cols; c0 += KC) {
      const int kc = (int)(cols - c0 < KC ? cols - c0 : KC);
      const int steps = kc / 32;
      f16x8 a[KU], bv[BI];
      // every load of the pass first, at clamped addresses (straight-line: the compiler keeps
      // them batched); rows of B past the pass are staged but never read
#pragma unroll
      for (int u = 0; u < KU; ++u) {
        const int s = w + u * NW < steps ? w + u * NW : steps - 1;   // clamped; zeroed below
        a[u] = *reinterpret_cast<const f16x8*>(in + m * ld + c0 + s * 32 + lk);
      }
#pragma unroll
      for (int q = 0; q < BI; ++q) {
        const int i = tid + q * kRowThreads, kk = i / (R / 8), r8 = (i % (R / 8)) * 8;
        bv[q] = *reinterpret_cast<const f16x8*>(wt + (c0 + (kk < kc ? kk : kc - 1)) * R + r8);
      }
      __builtin_amdgcn_sched_barrier(0);   // the pass's loads stay ahead of their first use
      __syncthreads();  // the previous pass has finished reading Bs
#pragma unroll
      for (int q = 0; q < BI; ++q) {
        const int i = tid + q * kRowThreads, kk = i / (R / 8), r8 = (i % (R / 8)) * 8;
        *reinterpret_cast<f16x8*>(Bs + kk * BLD + r8) = bv[q];
      }
      __syncthreads();
      {
#pragma unroll
        for (int u = 0; u < KU; ++u) {
          const int s0 = w + u * NW;
          const bool valid = s0 < steps;
          const int s = valid ? s0 : steps - 1;
#pragma unroll
          for (int e = 0; e < 8; ++e) a[u][e] = valid ? a[u][e] : (f16)0.0f;
#pragma unroll
          for (int b = 0; b < RB; ++b) {
            const f16* base = Bs + (s * 32 + trow) * BLD + 16 * b + tcol;
            const f16x4 lo = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(base)));
            const f16x4 hi = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (__attribute__((address_space(3))) i16x4*)(base + 4 * BLD)));
            const f16x8 bw = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[u], bw, acc[b], 0, 0, 0);
          }
        }
      }
    }
  }
#pragma unroll
  for (int b = 0; b < RB; ++b)
#pragma unroll
    for (int v = 0; v < 4; ++v) red[(w * 16 + 4 * (lane >> 4) + v) * R + 16 * b + lr] = acc[b][v];
  __syncthreads();
  for (int i = tid; i < 16 * R; i += kRowThreads) {
    const int rr = i / R, r = i % R;
    if (row0 + rr >= rows) continue;
    float sum = 0.0f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) sum += red[(ww * 16 + rr) * R + r];
    out[(row0 + rr) * R + r] = MODE == 0 ? dk_h(sum) : dk_h(__fmul_rn((float)dk_h(sum), scale));
  }
}

// Column reductions over every token row, one pass: out[c][r] = sum_m P[m][c] Q[m][r] (P =
// dropout(x) with the keep-mask when the job has one), then fp32(fp16(sum)) * scale, stored
// [c][r] or, transposed, [r][c].  A workgroup owns kSumCols columns of one job and all rows; its
// 8 waves take 32-row chunks in turn (chunk w, w + 8, ...), each with kSumDepth chunks of loads in
// flight, stage the chunk in a private LDS tile and run v_mfma_f32_16x16x32_f16 with both operands
// read M-contiguous by ds_read_b64_tr_b16: within each 16-lane group, lane 4a + b receives
// element b of the 4-element rows addressed by lanes a, a + 4, a + 8, a + 12, so lane l addressing
// row 8 (l / 16) + 4 h + (l % 16) / 4, column 4 (l % 4) receives rows 8 (l / 16) + 4 h + 0..3 of
// column l % 16, and two reads (h = 0, 1) give the 8 consecutive rows of the MFMA operand.  The
// waves' sums are added in wave order through LDS: the order of every sum is fixed, so results
// are deterministic, and there are no partial sums in memory and no second launch.
// Column blocks [bx0, next job's bx0) of the grid serve job j: the dB of each term (P = dY, Q = z)
// and the dA of each term (P = Xd, Q = dz) share one launch.
constexpr int kSumThreads = 512;
constexpr int kSumWaves = kSumThreads / 64;
// Measured on MI355X (q+v gradients at M = 2048, graph replay): 32 columns and 3 chunks in
// flight 17.5 us; 16 or 64 columns, or 5 chunks in flight, 19.7-24.4 us.
constexpr int kSumCols = 32;     // columns per workgroup
constexpr int kSumDepth = 3;     // 32-row chunks of loads in flight per wave
struct SumJob {
  const f16* P;
  int64_t ld;
  const uint8_t* mask;   // [rows][cols] keep-mask or null
  float ks;
  const f16* Q;          // [rows][R]
  float scale;
  float* out;
  int transpose;
  int64_t cols;
  int bx0;
};
constexpr int kMaxSumJobs = 2 * kMaxJobs;
struct SumJobs {
  SumJob j[kMaxSumJobs];
  int n;
};

// One column block of one job (see lora_colsum_kernel).  Every load is unconditional (rows past
// the end read the last row and are zeroed when staged), so the number of loads in flight is the
// same at every wait and the compiler's vmcnt waits count only the chunk being consumed.
template <int R, bool DROP>
__device__ __forceinline__ void colsum_block(const SumJob& J, int64_t rows, int b, uint8_t* lds) {
  const f16* __restrict__ P = J.P;
  const int64_t ld = J.ld;
  const uint8_t* __restrict__ mask = J.mask;
  const float ks = J.ks;
  const f16* __restrict__ Q = J.Q;
  const int64_t cols = J.cols;
  constexpr int PLD = kSumCols + 8;   // halves per staged P row
  constexpr int QLD = R + 8;          // halves per staged Q row
  constexpr int QL = R / 16;          // 16-byte Q pieces per lane per chunk
  constexpr int WAVE_LDS = 32 * PLD * 2 + 32 * QLD * 2;
  constexpr int D = kSumDepth;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  f16* Ps = reinterpret_cast<f16*>(lds + w * WAVE_LDS);
  f16* Qs = Ps + 32 * PLD;
  const int64_t c0 = (int64_t)(b - J.bx0) * kSumCols;
  const int64_t n_chunks = (rows + 31) / 32;
  const int64_t mine = n_chunks > w ? (n_chunks - w + kSumWaves - 1) / kSumWaves : 0;
  // this lane's pieces of a chunk: PL 16-byte P pieces (LPR lanes per row, rows l / LPR + RPL u,
  // 8 columns at 8 (l % LPR)) with their mask bytes, and QL 16-byte pieces of the Q rows
  constexpr int LPR = kSumCols / 8, RPL = 64 / LPR, PL = 32 / RPL;
  static_assert(PL * RPL == 32 && LPR * RPL == 64, "chunk layout");
  const int prow = lane / LPR, pc8 = 8 * (lane % LPR);
  f16x8 pv[D][PL], qv[D][QL];
  u32x2 mv[D][PL];
  auto row_of = [&](int64_t i, int r) {   // global row r of this wave's chunk i, clamped
    const int64_t m = 32 * (w + kSumWaves * i) + r;
    return m < rows ? m : rows - 1;
  };
  auto load = [&](int slot, int64_t i) {
#pragma unroll
    for (int u = 0; u < PL; ++u) {
      const int64_t m = row_of(i, prow + RPL * u);
      pv[slot][u] = *reinterpret_cast<const f16x8*>(P + m * ld + c0 + pc8);
      if (DROP) mv[slot][u] = *reinterpret_cast<const u32x2*>(mask + m * cols + c0 + pc8);
    }
#pragma unroll
    for (int u = 0; u < QL; ++u) {
      const int idx = lane + 64 * u;
      qv[slot][u] = *reinterpret_cast<const f16x8*>(Q + row_of(i, idx / (R / 8)) * R +
                                                    (idx % (R / 8)) * 8);
    }
  };
  const int trow = 8 * (lane >> 4) + ((lane & 15) >> 2), tcol = 4 * (lane & 3);
  auto tr8 = [&](const f16* base, int ldh) {
    const f16x4 lo = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(base)));
    const f16x4 hi = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4*)(base + 4 * ldh)));
    return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  };
  f32x4 acc[kSumCols / 16][R / 16];
#pragma unroll
  for (int cb = 0; cb < kSumCols / 16; ++cb)
#pragma unroll
    for (int rb = 0; rb < R / 16; ++rb) acc[cb][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto consume = [&](int slot, int64_t i) {
    const int64_t r0 = 32 * (w + kSumWaves * i);
    __builtin_amdgcn_wave_barrier();   // the previous chunk's transposing reads are done
#pragma unroll
    for (int u = 0; u < PL; ++u) {
      f16x8 v = pv[slot][u];
      const bool ok = r0 + prow + RPL * u < rows;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // the product is formed unconditionally, then selected (no branch per element)
        bool keep = ok;
        if (DROP) keep = keep && ((mv[slot][u][e >> 2] >> (8 * (e & 3))) & 0xffu) != 0;
        const f16 kept = DROP ? dk_h(__fmul_rn((float)v[e], ks)) : v[e];
        v[e] = keep ? kept : (f16)0.0f;
      }
      *reinterpret_cast<f16x8*>(Ps + (prow + RPL * u) * PLD + pc8) = v;
    }
#pragma unroll
    for (int u = 0; u < QL; ++u) {
      const int idx = lane + 64 * u, row = idx / (R / 8), r8 = (idx % (R / 8)) * 8;
      f16x8 q = qv[slot][u];
      if (r0 + row >= rows) {
#pragma unroll
        for (int e = 0; e < 8; ++e) q[e] = (f16)0.0f;
      }
      *reinterpret_cast<f16x8*>(Qs + row * QLD + r8) = q;
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int cb = 0; cb < kSumCols / 16; ++cb) {
      const f16x8 a = tr8(Ps + trow * PLD + 16 * cb + tcol, PLD);
#pragma unroll
      for (int rb = 0; rb < R / 16; ++rb) {
        const f16x8 b = tr8(Qs + trow * QLD + 16 * rb + tcol, QLD);
        acc[cb][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[cb][rb], 0, 0, 0);
      }
    }
  };
  // D chunks in flight: the loads of chunk i + D - 1 (clamped to the wave's last chunk) go out
  // before chunk i is consumed; slots rotate with the unrolled index
  if (mine > 0) {
#pragma unroll
    for (int s = 0; s < D - 1; ++s) load(s, s < mine ? s : mine - 1);
    for (int64_t i0 = 0; i0 < mine; i0 += D) {
#pragma unroll
      for (int s = 0; s < D; ++s) {
        const int64_t i = i0 + s;
        const int64_t nx = i + D - 1 < mine ? i + D - 1 : mine - 1;
        load((s + D - 1) % D, nx);
        __builtin_amdgcn_sched_barrier(0);   // the next chunk's loads go out before this one's use
        if (i < mine) consume(s, i);
      }
    }
  }
  // the waves' sums in wave order, one rank block at a time; result register v of lane l holds
  // column 16 cb + 4 (l / 16) + v, rank 16 rb + l % 16
  __syncthreads();   // every wave is done with its staging tile
  float* red = reinterpret_cast<float*>(lds);
#pragma unroll
  for (int rb = 0; rb < R / 16; ++rb) {
#pragma unroll
    for (int cb = 0; cb < kSumCols / 16; ++cb)
#pragma unroll
      for (int v = 0; v < 4; ++v)
        red[(w * kSumCols + 16 * cb + 4 * (lane >> 4) + v) * 16 + (lane & 15)] = acc[cb][rb][v];
    __syncthreads();
    for (int t = tid; t < kSumCols * 16; t += kSumThreads) {
      const int c = t / 16, r = t % 16;
      float s = 0.0f;
#pragma unroll
      for (int ww = 0; ww < kSumWaves; ++ww) s += red[(ww * kSumCols + c) * 16 + r];
      const float v = __fmul_rn((float)dk_h(s), J.scale);
      const int64_t col = c0 + c;
      if (col < cols) {
        if (J.transpose) J.out[(int64_t)(16 * rb + r) * cols + col] = v;
        else J.out[col * R + 16 * rb + r] = v;
      }
    }
    __syncthreads();
  }
}

template <int R>
__global__ __launch_bounds__(kSumThreads) void lora_colsum_kernel(SumJobs jobs, int64_t rows) {
  // workgroups are dealt to the 8 XCDs round-robin: give each XCD a contiguous run of column
  // blocks, so the two 64-byte halves of a row's 128-byte line (neighbouring blocks) share an L2
  int b = blockIdx.x;
  if ((gridDim.x & 7) == 0) b = (b & 7) * (gridDim.x >> 3) + (b >> 3);
  int jb = 0;
#pragma unroll
  for (int q = 1; q < kMaxSumJobs; ++q)
    if (q < jobs.n && b >= jobs.j[q].bx0) jb = q;
  constexpr int WAVE_LDS = 32 * (kSumCols + 8) * 2 + 32 * (R + 8) * 2;
  constexpr int RED = kSumWaves * kSumCols * 16 * 4;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kSumWaves * WAVE_LDS > RED ? kSumWaves * WAVE_LDS : RED];
  if (jobs.j[jb].mask) colsum_block<R, true>(jobs.j[jb], rows, b, lds);
  else colsum_block<R, false>(jobs.j[jb], rows, b, lds);
}

template <int MODE, bool MASKED>
int rows_launch(int64_t R, hipStream_t stream, const RowsJobs& jobs, int n_jobs, int64_t rows) {
  const dim3 grid((unsigned)(n_jobs * ((rows + kRowTile - 1) / kRowTile))), block(kRowThreads);
  switch (R) {
    case 16: hipLaunchKernelGGL((lora_rows_kernel<16, MODE, MASKED>), grid, block, 0, stream, jobs, rows); break;
    case 32: hipLaunchKernelGGL((lora_rows_kernel<32, MODE, MASKED>), grid, block, 0, stream, jobs, rows); break;
    case 48: hipLaunchKernelGGL((lora_rows_kernel<48, MODE, MASKED>), grid, block, 0, stream, jobs, rows); break;
    case 64: hipLaunchKernelGGL((lora_rows_kernel<64, MODE, MASKED>), grid, block, 0, stream, jobs, rows); break;
    default: return DK_ERR_INVALID;
  }
  DK_CHECK_LAUNCH();
  return 0;
}

int colsum_launch(int64_t R, hipStream_t stream, SumJobs jobs, int64_t rows) {
  int bx = 0;
  for (int q = 0; q < jobs.n; ++q) {
    jobs.j[q].bx0 = bx;
    bx += (int)((jobs.j[q].cols + kSumCols - 1) / kSumCols);
  }
  const dim3 grid((unsigned)bx), block(kSumThreads);
  switch (R) {
    case 16: hipLaunchKernelGGL((lora_colsum_kernel<16>), grid, block, 0, stream, jobs, rows); break;
    case 32: hipLaunchKernelGGL((lora_colsum_kernel<32>), grid, block, 0, stream, jobs, rows); break;
    case 48: hipLaunchKernelGGL((lora_colsum_kernel<48>), grid, block, 0, stream, jobs, rows); break;
    case 64: hipLaunchKernelGGL((lora_colsum_kernel<64>), grid, block, 0, stream, jobs, rows); break;
    default: return DK_ERR_INVALID;
  }
  DK_CHECK_LAUNCH();
  return 0;
}

bool rank_ok(int64_t r) { return r >= 16 && r <= 64 && r % 16 == 0; }

}  // namespace

extern "C" int dk_lora_down_multi(const void* x, int64_t m, int64_t k, int64_t rank,
                                  const dk_lora_down_term* terms, int n_terms, hipStream_t stream) {
  // (zero-element tensors have null data pointers: the inputs and z are required only with rows)
  if (m < 0 || k <= 0 || k % 32 || !rank_ok(rank) || !terms || n_terms < 1 || n_terms > kMaxJobs)
    return DK_ERR_INVALID;
  if (!dk_aligned(x, 16)) return DK_ERR_ALIGN;
  int masked = 0;
  for (int t = 0; t < n_terms; ++t) {
    const dk_lora_down_term& u = terms[t];
    if (m > 0 && (!u.a || !u.z || !(u.x ? u.x : x))) return DK_ERR_INVALID;
    if (!dk_aligned(u.a, 16) || !dk_aligned(u.x, 16) || (u.mask && !dk_aligned(u.mask, 8)))
      return DK_ERR_ALIGN;
    masked += u.mask != nullptr;
  }
  if (m == 0) return 0;
  auto job = [&](const dk_lora_down_term& u) {
    return RowsJob{(const f16*)(u.x ? u.x : x), k, u.mask, u.mask ? u.keep_scale : 1.0f,
                   (const f16*)u.a, 1.0f, (f16*)u.z, k};
  };
  if (masked == 0 || masked == n_terms) {
    RowsJobs jobs = {};
    for (int t = 0; t < n_terms; ++t) jobs.j[t] = job(terms[t]);
    return masked ? rows_launch<0, true>(rank, stream, jobs, n_terms, m)
                  : rows_launch<0, false>(rank, stream, jobs, n_terms, m);
  }
  for (int t = 0; t < n_terms; ++t) {   // masked and unmasked terms: one launch each
    RowsJobs jobs = {};
    jobs.j[0] = job(terms[t]);
    const int e = terms[t].mask ? rows_launch<0, true>(rank, stream, jobs, 1, m)
                                : rows_launch<0, false>(rank, stream, jobs, 1, m);
    if (e) return e;
  }
  return 0;
}

extern "C" int dk_lora_down(const void* x, const uint8_t* mask, float keep_scale, const void* a,
                            void* z, int64_t m, int64_t k, int64_t rank, hipStream_t stream) {
  const dk_lora_down_term t = {mask, keep_scale, a, z, nullptr};
  return dk_lora_down_multi(x, m, k, rank, &t, 1, stream);
}

extern "C" int64_t dk_lora_grads_multi_workspace(int64_t, int64_t, int64_t, const int64_t*, int) {
  return 0;
}

extern "C" int64_t dk_lora_grads_workspace(int64_t, int64_t, int64_t, int64_t) { return 0; }

extern "C" int dk_lora_grads_multi(const void* x, int64_t m, int64_t k, int64_t rank,
                                   const dk_lora_grads_term* terms, int n_terms, void*, int64_t,
                                   hipStream_t stream) {
  if (m < 0 || k <= 0 || k % 32 || !rank_ok(rank) || !terms || n_terms < 1 || n_terms > kMaxJobs)
    return DK_ERR_INVALID;
  if (!dk_aligned(x, 16)) return DK_ERR_ALIGN;
  for (int t = 0; t < n_terms; ++t) {
    const dk_lora_grads_term& u = terms[t];
    // zero-element tensors have null data pointers: the row operands are required only with rows
    if (u.n_out <= 0 || u.n_out % 32 || !u.lora_b || !u.da || !u.db || u.lddy < u.n_out ||
        (m > 0 && (!u.dy || !u.z || !u.dz || !(u.x ? u.x : x))))
      return DK_ERR_INVALID;
    if (!dk_aligned(u.dy, 16) || u.lddy % 8 || !dk_aligned(u.lora_b, 16) || !dk_aligned(u.x, 16) ||
        (u.mask && !dk_aligned(u.mask, 8)))
      return DK_ERR_ALIGN;
  }
  // dz = fp16(fp16(dY B) * s)
  if (m > 0) {
    RowsJobs rj = {};
    for (int t = 0; t < n_terms; ++t) {
      const dk_lora_grads_term& u = terms[t];
      rj.j[t] = RowsJob{(const f16*)u.dy, u.lddy, nullptr, 1.0f, (const f16*)u.lora_b,
                        u.lora_scale, (f16*)u.dz, u.n_out};
    }
    const int e = rows_launch<1, false>(rank, stream, rj, n_terms, m);
    if (e) return e;
  }
  // one launch: dB = fp32(fp16(dY^T z)) * s of every term, then dA = fp32(fp16(dz^T Xd)), Xd the
  // term's input with its keep-mask (zero rows: both are zero)
  SumJobs sj = {};
  sj.n = 2 * n_terms;
  for (int t = 0; t < n_terms; ++t) {
    const dk_lora_grads_term& u = terms[t];
    sj.j[t] = SumJob{(const f16*)u.dy, u.lddy, nullptr, 1.0f, (const f16*)u.z, u.lora_scale,
                     u.db, 0, u.n_out, 0};
    sj.j[n_terms + t] = SumJob{(const f16*)(u.x ? u.x : x), k, u.mask,
                               u.mask ? u.keep_scale : 1.0f, (const f16*)u.dz, 1.0f, u.da, 1, k, 0};
  }
  return colsum_launch(rank, stream, sj, m);
}

extern "C" int dk_lora_grads(const void* dy, int64_t lddy, const void* z, const void* x,
                             const uint8_t* mask, float keep_scale, const void* lora_b,
                             float lora_scale, int64_t m, int64_t n_out, int64_t k, int64_t rank,
                             float* da, float* db, void* dz, void* ws, int64_t ws_bytes,
                             hipStream_t stream) {
  const dk_lora_grads_term t = {dy, lddy, n_out, z, lora_b, lora_scale, mask, keep_scale, da, db,
                                dz, nullptr};
  return dk_lora_grads_multi(x, m, k, rank, &t, 1, ws, ws_bytes, stream);
}
