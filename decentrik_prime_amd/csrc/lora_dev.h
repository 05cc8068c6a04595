// Device code of the LoRA column sums (dB and dA over every token row), shared by their own
// launch (lora.hip) and by the dX GEMM launches that carry them on idle CUs (hgemm.hip).
#pragma once
#include "dk_common.h"

namespace dk {

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
constexpr int kMaxSumJobs = 4;   // dB and dA of two LoRA terms
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

// Bytes of LDS colsum_run<R> needs (the per-wave staging tiles, or the cross-wave sums).
template <int R>
constexpr int colsum_lds_bytes() {
  return kSumWaves * (32 * (kSumCols + 8) * 2 + 32 * (R + 8) * 2) > kSumWaves * kSumCols * 16 * 4
             ? kSumWaves * (32 * (kSumCols + 8) * 2 + 32 * (R + 8) * 2)
             : kSumWaves * kSumCols * 16 * 4;
}

// Column block j of a grid of n blocks whose first workgroup has index base.  Workgroups are
// dealt to the 8 XCDs round-robin; with n a multiple of 8 each XCD gets a contiguous run of
// column blocks, so the two 64-byte halves of a row's 128-byte line (neighbouring blocks) share
// an L2.
__device__ __forceinline__ int colsum_block_of(int j, int n, int base) {
  return (n & 7) == 0 ? ((base + j) & 7) * (n >> 3) + (j >> 3) : j;
}

// Column block b of the jobs (the job whose [bx0, next bx0) holds b), with lds of
// colsum_lds_bytes<R>() bytes.
template <int R>
__device__ __forceinline__ void colsum_run(const SumJobs& jobs, int64_t rows, int b, uint8_t* lds) {
  int jb = 0;
#pragma unroll
  for (int q = 1; q < kMaxSumJobs; ++q)
    if (q < jobs.n && b >= jobs.j[q].bx0) jb = q;
  if (jobs.j[jb].mask) colsum_block<R, true>(jobs.j[jb], rows, b, lds);
  else colsum_block<R, false>(jobs.j[jb], rows, b, lds);
}

// Column sums a dX GEMM launch carries: `wgs` workgroups (the jobs' column blocks) after its
// tiles, rank 16; wgs 0: none.
struct SideSums {
  SumJobs jobs;
  int64_t rows;
  int wgs;
};

// The column-sum jobs of dk_lora_grads_multi's terms (dB of each term, then dA of each), with
// their column blocks numbered (bx0) and the total in *blocks; DK_ERR_* on bad arguments
// (lora.hip).
int lora_sum_jobs(const void* x, int64_t m, int64_t k, int64_t rank,
                  const dk_lora_grads_term* terms, int n_terms, SumJobs* jobs, int* blocks);
// The column sums as a launch of their own (lora.hip).
int lora_sums_launch(int64_t rank, const SumJobs& jobs, int blocks, int64_t rows,
                     hipStream_t stream);

}  // namespace dk
