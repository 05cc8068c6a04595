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
#include "lora_dev.h"
#include "nf4_dev.h"

using namespace dk;

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

// Row block `blk` of the jobs (the body of lora_rows_kernel, also run by the first workgroups of
// lora_down_dequant_kernel).  NWP: the workgroup's waves; with fewer than the 8 of the K split
// (MODE 0 only), wave w runs the split's waves w, w + NWP, ... one after the other, so every sum
// keeps the 8-wave kernel's order.
template <int R, int MODE, bool MASKED, int NWP = kRowThreads / 64>
__device__ __forceinline__ void rows_block(const RowsJobs& jobs, int64_t rows, int blk) {
  const int64_t per_job = (rows + kRowTile - 1) / kRowTile;
  const RowsJob& J = jobs.j[blk / per_job];
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
  static_assert(NW % NWP == 0 && (MODE == 0 || NWP == NW), "waves");
  __shared__ float red[NW * 16 * R];
  __shared__ __attribute__((aligned(16))) f16 Bs[MODE == 1 ? KC * BLD : 8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t row0 = (int64_t)(blk % per_job) * kRowTile;
  const int lr = lane & 15, lk = 8 * (lane >> 4);
  const int64_t m = row0 + lr < rows ? row0 + lr : rows - 1;   // clamped: its sums are not stored
  const int trow = 8 * (lane >> 4) + ((lane & 15) >> 2), tcol = 4 * (lane & 3);
  f32x4 acc[RB];
#pragma unroll
  for (int b = 0; b < RB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (MODE == 0) {
    const int64_t steps = cols / 32;
    for (int vw = w; vw < NW; vw += NWP) {   // the split's wave vw
    if (vw != w) {
#pragma unroll
      for (int b = 0; b < RB; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    for (int64_t s0 = vw; s0 < steps; s0 += NW * kBatch) {
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
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[(vw * 16 + 4 * (lane >> 4) + v) * R + 16 * b + lr] = acc[b][v];
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
  if (MODE == 1) {
#pragma unroll
    for (int b = 0; b < RB; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) red[(w * 16 + 4 * (lane >> 4) + v) * R + 16 * b + lr] = acc[b][v];
  }
  __syncthreads();
  for (int i = tid; i < 16 * R; i += NWP * 64) {
    const int rr = i / R, r = i % R;
    if (row0 + rr >= rows) continue;
    float sum = 0.0f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) sum += red[(ww * 16 + rr) * R + r];
    out[(row0 + rr) * R + r] = MODE == 0 ? dk_h(sum) : dk_h(__fmul_rn((float)dk_h(sum), scale));
  }
}

template <int R, int MODE, bool MASKED>
__global__ __launch_bounds__(kRowThreads) void lora_rows_kernel(RowsJobs jobs, int64_t rows) {
  rows_block<R, MODE, MASKED>(jobs, rows, (int)blockIdx.x);
}

// The LoRA downs (MODE 0 row blocks, workgroups [0, row_wgs)) and a dequant of second-level
// blocks [dq.sb0, dq.sb1) (the workgroups after them, one block per wave, converted and stored
// as nf4_dequant_kernel does) in one launch: both memory-bound and independent, so the row
// blocks' load latency overlaps the dequant's stream instead of adding a launch of its own.
constexpr int kDqLoraThreads = 256;   // the standalone dequant's workgroup (4 waves)
template <int R, bool MASKED>
__global__ __launch_bounds__(kDqLoraThreads) void lora_down_dequant_kernel(RowsJobs jobs,
                                                                           int64_t rows,
                                                                           int row_wgs,
                                                                           SideDequant dq) {
  if ((int)blockIdx.x < row_wgs) {
    rows_block<R, 0, MASKED, kDqLoraThreads / 64>(jobs, rows, (int)blockIdx.x);
    return;
  }
  __shared__ float lut[16];
  __shared__ float c2[256];
  const int lane = threadIdx.x & 63;
  const int64_t sb = dq.sb0 + (int64_t)((int)blockIdx.x - row_wgs) * (kDqLoraThreads / 64) +
                     __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t last = dq.sb1 * (DK_ELEMS_PER_SB / 8) - 1;
  const uint32_t* packed = reinterpret_cast<const uint32_t*>(dq.packed);
  const float c2v = dq.code2[threadIdx.x & 255], lutv = dq.nf4[threadIdx.x & 15];
  WaveLoads L;
  if (sb < dq.sb1) dq_wave_load(packed, dq.qabs, dq.scale2, dq.offset2, sb * 2048, last, lane, L);
  if (threadIdx.x < 256) c2[threadIdx.x] = c2v;
  if (threadIdx.x < 16) lut[threadIdx.x] = lutv;
  __syncthreads();
  if (sb < dq.sb1) dq_wave_store<false>(L, c2, lut, dq.out, sb * 2048, last, lane);
}

template <int R>
__global__ __launch_bounds__(kSumThreads) void lora_colsum_kernel(SumJobs jobs, int64_t rows) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[colsum_lds_bytes<R>()];
  colsum_run<R>(jobs, rows, colsum_block_of((int)blockIdx.x, (int)gridDim.x, 0), lds);
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

namespace {
template <int R>
void down_dequant_launch(bool masked, dim3 grid, dim3 block, hipStream_t stream,
                         const RowsJobs& jobs, int64_t m, int rw, const SideDequant& dq) {
  if (masked)
    hipLaunchKernelGGL((lora_down_dequant_kernel<R, true>), grid, block, 0, stream, jobs, m, rw, dq);
  else
    hipLaunchKernelGGL((lora_down_dequant_kernel<R, false>), grid, block, 0, stream, jobs, m, rw, dq);
}
}  // namespace

extern "C" int dk_lora_down_multi_dequant(const void* x, int64_t m, int64_t k, int64_t rank,
                                          const dk_lora_down_term* terms, int n_terms,
                                          const dk_side_dequant* side, hipStream_t stream) {
  // the dequant's description, checked as a GEMM's carried dequant is (its wgs is not used)
  if (!side || side->sb0 < 0 || side->sb1 < side->sb0) return DK_ERR_INVALID;
  if (side->sb1 > side->sb0 && (!side->packed || !side->qabs || !side->scale2 || !side->offset2 ||
                                !side->code2 || !side->nf4 || !side->out))
    return DK_ERR_INVALID;
  if (side->sb1 > side->sb0 && (!dk_aligned(side->packed, 16) || !dk_aligned(side->out, 16)))
    return DK_ERR_ALIGN;
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
  const int64_t n_sb = side->sb1 - side->sb0;
  const int64_t dq_wgs = (n_sb + kDqLoraThreads / 64 - 1) / (kDqLoraThreads / 64);
  const int64_t row_wgs = n_terms * ((m + kRowTile - 1) / kRowTile);
  if (m == 0 || n_sb == 0 || (masked != 0 && masked != n_terms) || row_wgs + dq_wgs > 0x7fffffff) {
    // nothing to share a launch with, or terms that need launches of their own: one call each
    if (n_sb > 0) {
      if (int e = dk_nf4_dequant(side->packed + side->sb0 * (DK_ELEMS_PER_SB / 2),
                                 side->qabs + side->sb0 * (DK_ELEMS_PER_SB / 64),
                                 side->scale2 + side->sb0, side->offset2 + side->sb0, side->code2,
                                 side->nf4, reinterpret_cast<f16*>(side->out) +
                                                side->sb0 * DK_ELEMS_PER_SB,
                                 n_sb * (DK_ELEMS_PER_SB / 64), stream))
        return e;
    }
    return m > 0 ? dk_lora_down_multi(x, m, k, rank, terms, n_terms, stream) : 0;
  }
  RowsJobs jobs = {};
  for (int t = 0; t < n_terms; ++t) {
    const dk_lora_down_term& u = terms[t];
    jobs.j[t] = RowsJob{(const f16*)(u.x ? u.x : x), k, u.mask, u.mask ? u.keep_scale : 1.0f,
                        (const f16*)u.a, 1.0f, (f16*)u.z, k};
  }
  SideDequant dq{reinterpret_cast<const u32x4*>(side->packed), side->qabs, side->scale2,
                 side->offset2, side->code2, side->nf4, reinterpret_cast<u32x4*>(side->out),
                 side->sb0, side->sb1, 0};
  const dim3 grid((unsigned)(row_wgs + dq_wgs)), block(kDqLoraThreads);
  const int rw = (int)row_wgs;
  switch (rank) {
    case 16: down_dequant_launch<16>(masked > 0, grid, block, stream, jobs, m, rw, dq); break;
    case 32: down_dequant_launch<32>(masked > 0, grid, block, stream, jobs, m, rw, dq); break;
    case 48: down_dequant_launch<48>(masked > 0, grid, block, stream, jobs, m, rw, dq); break;
    case 64: down_dequant_launch<64>(masked > 0, grid, block, stream, jobs, m, rw, dq); break;
    default: return DK_ERR_INVALID;
  }
  DK_CHECK_LAUNCH();
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

namespace {

// Arguments of dk_lora_grads_multi and its two halves.
int grads_args(const void* x, int64_t m, int64_t k, int64_t rank, const dk_lora_grads_term* terms,
               int n_terms) {
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
  return 0;
}

}  // namespace

namespace dk {

int lora_sum_jobs(const void* x, int64_t m, int64_t k, int64_t rank,
                  const dk_lora_grads_term* terms, int n_terms, SumJobs* jobs, int* blocks) {
  if (int e = grads_args(x, m, k, rank, terms, n_terms)) return e;
  // dB = fp32(fp16(dY^T z)) * s of every term, then dA = fp32(fp16(dz^T Xd)), Xd the term's input
  // with its keep-mask (zero rows: both are zero)
  SumJobs& sj = *jobs;
  sj = SumJobs{};
  sj.n = 2 * n_terms;
  for (int t = 0; t < n_terms; ++t) {
    const dk_lora_grads_term& u = terms[t];
    sj.j[t] = SumJob{(const f16*)u.dy, u.lddy, nullptr, 1.0f, (const f16*)u.z, u.lora_scale,
                     u.db, 0, u.n_out, 0};
    sj.j[n_terms + t] = SumJob{(const f16*)(u.x ? u.x : x), k, u.mask,
                               u.mask ? u.keep_scale : 1.0f, (const f16*)u.dz, 1.0f, u.da, 1, k, 0};
  }
  int bx = 0;
  for (int q = 0; q < sj.n; ++q) {
    sj.j[q].bx0 = bx;
    bx += (int)((sj.j[q].cols + kSumCols - 1) / kSumCols);
  }
  *blocks = bx;
  return 0;
}

int lora_sums_launch(int64_t rank, const SumJobs& jobs, int blocks, int64_t rows,
                     hipStream_t stream) {
  const dim3 grid((unsigned)blocks), block(kSumThreads);
  switch (rank) {
    case 16: hipLaunchKernelGGL((lora_colsum_kernel<16>), grid, block, 0, stream, jobs, rows); break;
    case 32: hipLaunchKernelGGL((lora_colsum_kernel<32>), grid, block, 0, stream, jobs, rows); break;
    case 48: hipLaunchKernelGGL((lora_colsum_kernel<48>), grid, block, 0, stream, jobs, rows); break;
    case 64: hipLaunchKernelGGL((lora_colsum_kernel<64>), grid, block, 0, stream, jobs, rows); break;
    default: return DK_ERR_INVALID;
  }
  DK_CHECK_LAUNCH();
  return 0;
}

}  // namespace dk

extern "C" int dk_lora_dz_multi(const void* x, int64_t m, int64_t k, int64_t rank,
                                const dk_lora_grads_term* terms, int n_terms, hipStream_t stream) {
  if (int e = grads_args(x, m, k, rank, terms, n_terms)) return e;
  if (m == 0) return 0;
  // dz = fp16(fp16(dY B) * s)
  RowsJobs rj = {};
  for (int t = 0; t < n_terms; ++t) {
    const dk_lora_grads_term& u = terms[t];
    rj.j[t] = RowsJob{(const f16*)u.dy, u.lddy, nullptr, 1.0f, (const f16*)u.lora_b,
                      u.lora_scale, (f16*)u.dz, u.n_out};
  }
  return rows_launch<1, false>(rank, stream, rj, n_terms, m);
}

extern "C" int dk_lora_grads_multi(const void* x, int64_t m, int64_t k, int64_t rank,
                                   const dk_lora_grads_term* terms, int n_terms, void*, int64_t,
                                   hipStream_t stream) {
  SumJobs sj;
  int blocks = 0;
  if (int e = lora_sum_jobs(x, m, k, rank, terms, n_terms, &sj, &blocks)) return e;
  if (int e = dk_lora_dz_multi(x, m, k, rank, terms, n_terms, stream)) return e;
  return lora_sums_launch(rank, sj, blocks, m, stream);
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
