// NF4 double-quantised weights on gfx950: the HBM-rate dequant and the blockwise quantiser.
//
// Dequant (replaces solution/k_nf4.py:40-57).  Each wave converts one second-level block (2048
// packed dwords of 8 weights, 16384 weights) with nf4_dev.h's dq_wave_load / dq_wave_store: every
// load instruction of the wave reads 256 contiguous bytes and every store instruction writes the
// 64 lanes' 16-byte results, 1 KiB contiguous, straight from registers (no LDS staging, no
// barrier before the stores).  A workgroup's four waves fill the two LDS tables (NF4 values and
// the second-level codes) while their loads are in flight.  HBM traffic: 2.516 bytes per weight
// (0.5 packed + 1/64 code + 8/16384 scale/offset in, 2 out).
#include "nf4_dev.h"

using dk::kWaveDwords;
using dk::WaveLoads;
using dk::dq_wave_load;
using dk::dq_wave_store;

namespace {

// 32 dwords per lane (256 weights) in 256-thread workgroups, 714 per Qwen2.5-1.5B layer: measured
// on MI355X over 28 layer buffers (graph-replayed, gaps included) 5.5-5.6 TB/s, against 4.8-5.0
// for the former one-quad-per-lane kernel with LDS-staged stores, 5.1-5.2 for 8 or 16 dwords per
// lane (16 with 512 threads), 4.8-5.1 for 8 or 16 with 1024 threads and 4.9 for 64; cached
// instead of non-temporal loads of the packed bytes cost 6-7 %.  With the conversion replaced by
// a plain copy of the packed words, 8 dwords per lane ran at the same 5.2 TB/s: more bytes in
// flight per wave, not less arithmetic, is what raised the rate (writes alone reach 6.9 TB/s)
constexpr int kDqThreads = 256;
constexpr int kDqWgDwords = kDqThreads * kWaveDwords;
static_assert(kDqThreads == 256, "one code2 entry per thread");

__global__ __launch_bounds__(kDqThreads) void nf4_dequant_kernel(
    const uint32_t* __restrict__ packed, const uint8_t* __restrict__ qabs,
    const float* __restrict__ scale2, const float* __restrict__ offset2,
    const float* __restrict__ code2, const float* __restrict__ nf4, u32x4* __restrict__ out,
    int64_t n_dwords) {
  __shared__ float lut[16];
  __shared__ float c2[256];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t d_wave = (int64_t)blockIdx.x * kDqWgDwords + wave * 64 * kWaveDwords;
  const int64_t last = n_dwords - 1;
  // the tables' loads first (the LDS fill waits only for them), then the codes and the dwords
  const float c2v = code2[threadIdx.x];
  const float lutv = nf4[threadIdx.x & 15];
  WaveLoads L;
  dq_wave_load(packed, qabs, scale2, offset2, d_wave, last, lane, L);
  c2[threadIdx.x] = c2v;
  if (threadIdx.x < 16) lut[threadIdx.x] = lutv;
  __syncthreads();
  dq_wave_store<false>(L, c2, lut, out, d_wave, last, lane);
}

// ---------------------------------------------------------------------------------------------
// Quantiser.  Pass 1: one thread per 64-weight block computes absmax = max|w|, the NF4 codes of
// w * fp32(1/absmax) (code = number of fp32 midpoints between consecutive NF4 values strictly
// below it; an all-zero block gives code 7) and the packed bytes, and adds absmax to an exact
// integer sum in units of 2^-24.  Pass 2: one 256-thread block per second-level block
// subtracts offset = fp32(sum / n) and quantises each absmax against the 256-entry code table
// (nearest entry, ties to the lower index) after normalising by the block's max magnitude.

constexpr int kQThreads = 256;

__global__ void zero_u64_kernel(uint64_t* p) { *p = 0; }

__global__ __launch_bounds__(kQThreads) void nf4_quant_pass1(
    const f16x8* __restrict__ w, const float* __restrict__ nf4, u32x4* __restrict__ packed,
    float* __restrict__ absmax_out, uint64_t* __restrict__ sum, int64_t n_qblocks) {
  __shared__ float mid[15];
  __shared__ uint64_t red[kQThreads / 64];
  if (threadIdx.x < 15) {
    mid[threadIdx.x] = __fmul_rn(__fadd_rn(nf4[threadIdx.x], nf4[threadIdx.x + 1]), 0.5f);
  }
  __syncthreads();
  const int64_t q = (int64_t)blockIdx.x * kQThreads + threadIdx.x;
  uint64_t units = 0;
  if (q < n_qblocks) {
    f16x8 v[8];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[i] = w[q * 8 + i];
#pragma unroll
      for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf((float)v[i][e]));
    }
    const float inv = amax != 0.0f ? __fdiv_rn(1.0f, amax) : 0.0f;
    uint32_t words[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = __fmul_rn((float)v[i][e], inv);
        uint32_t code = 0;
#pragma unroll
        for (int t = 0; t < 15; ++t) code += (x > mid[t]) ? 1u : 0u;
        // element 2j -> high nibble of byte j
        const int byte = e >> 1;
        const int shift = 8 * byte + ((e & 1) ? 0 : 4);
        word |= code << shift;
      }
      words[i] = word;
    }
    packed[q * 2] = u32x4{words[0], words[1], words[2], words[3]};
    packed[q * 2 + 1] = u32x4{words[4], words[5], words[6], words[7]};
    absmax_out[q] = amax;
    units = (uint64_t)ldexpf(amax, 24);  // exact: amax is an fp16 magnitude, a multiple of 2^-24
  }
  // block sum of units, then one atomic per block (integer: order independent)
  for (int off = 32; off > 0; off >>= 1) units += __shfl_xor(units, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = units;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint64_t s = 0;
    for (int i = 0; i < kQThreads / 64; ++i) s += red[i];
    atomicAdd((unsigned long long*)sum, (unsigned long long)s);
  }
}

__global__ __launch_bounds__(kQThreads) void nf4_quant_pass2(
    const float* __restrict__ absmax, const float* __restrict__ code2,
    const uint64_t* __restrict__ sum, uint8_t* __restrict__ qabs, float* __restrict__ scale2,
    float* __restrict__ offset2, int64_t n_qblocks) {
  __shared__ float table[256];
  __shared__ float red[kQThreads / 64];
  table[threadIdx.x] = code2[threadIdx.x];
  const float offset = (float)(((double)(*sum) / (double)n_qblocks) * 0x1p-24);
  const int64_t q = (int64_t)blockIdx.x * kQThreads + threadIdx.x;
  const float v = __fsub_rn(absmax[q], offset);
  float m = fabsf(v);
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float a2 = red[0];
  for (int i = 1; i < kQThreads / 64; ++i) a2 = fmaxf(a2, red[i]);
  const float inv = a2 != 0.0f ? __fdiv_rn(1.0f, a2) : 0.0f;
  const float y = __fmul_rn(v, inv);
  // count = number of table entries <= y (the table is sorted ascending)
  int lo = 0, hi = 256;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (table[mid] <= y) lo = mid + 1; else hi = mid;
  }
  int i0 = lo - 1;
  if (i0 < 0) i0 = 0;
  const int i1 = i0 + 1 < 256 ? i0 + 1 : 255;
  const float d_hi = __fsub_rn(table[i1], y);
  const float d_lo = __fsub_rn(y, table[i0]);
  qabs[q] = (uint8_t)(d_hi < d_lo ? i1 : i0);
  if (threadIdx.x == 0) {
    scale2[blockIdx.x] = a2;
    offset2[blockIdx.x] = offset;
  }
}

}  // namespace

extern "C" int dk_nf4_dequant(const uint8_t* packed, const uint8_t* qabs, const float* scale2,
                              const float* offset2, const float* code2, const float* nf4,
                              void* out_f16, int64_t n_qblocks, hipStream_t stream) {
  if (n_qblocks < 0) return DK_ERR_INVALID;
  if (n_qblocks == 0) return 0;
  if (!packed || !qabs || !scale2 || !offset2 || !code2 || !nf4 || !out_f16) return DK_ERR_INVALID;
  if (!dk_aligned(packed, 16) || !dk_aligned(out_f16, 16)) return DK_ERR_ALIGN;
  const int64_t n_dwords = n_qblocks * 8;
  const int64_t grid = (n_dwords + kDqWgDwords - 1) / kDqWgDwords;
  if (grid > 0x7fffffff) return DK_ERR_INVALID;
  hipLaunchKernelGGL(nf4_dequant_kernel, dim3((unsigned)grid), dim3(kDqThreads), 0, stream,
                     reinterpret_cast<const uint32_t*>(packed), qabs, scale2, offset2, code2, nf4,
                     reinterpret_cast<u32x4*>(out_f16), n_dwords);
  DK_CHECK_LAUNCH();
  return 0;
}

extern "C" int dk_nf4_quantize(const void* w_f16, int64_t numel, const float* code2,
                               const float* nf4, uint8_t* packed, uint8_t* qabs, float* scale2,
                               float* offset2, float* absmax_ws, uint64_t* sum_ws,
                               hipStream_t stream) {
  if (numel <= 0 || numel % DK_ELEMS_PER_SB) return DK_ERR_INVALID;
  if (!w_f16 || !code2 || !nf4 || !packed || !qabs || !scale2 || !offset2 || !absmax_ws || !sum_ws)
    return DK_ERR_INVALID;
  if (!dk_aligned(w_f16, 16) || !dk_aligned(packed, 16) || !dk_aligned(sum_ws, 8))
    return DK_ERR_ALIGN;
  const int64_t nq = numel / DK_QBLOCK;
  hipLaunchKernelGGL(zero_u64_kernel, dim3(1), dim3(1), 0, stream, sum_ws);
  DK_CHECK_LAUNCH();
  hipLaunchKernelGGL(nf4_quant_pass1, dim3((unsigned)((nq + kQThreads - 1) / kQThreads)),
                     dim3(kQThreads), 0, stream, reinterpret_cast<const f16x8*>(w_f16), nf4,
                     reinterpret_cast<u32x4*>(packed), absmax_ws, sum_ws, nq);
  DK_CHECK_LAUNCH();
  hipLaunchKernelGGL(nf4_quant_pass2, dim3((unsigned)(nq / DK_QBLOCK2)), dim3(kQThreads), 0, stream,
                     absmax_ws, code2, sum_ws, qabs, scale2, offset2, nq);
  DK_CHECK_LAUNCH();
  return 0;
}
