// NF4 dequant device code shared by the standalone dequant kernel (nf4.hip) and the dequant work
// the GEMM launches carry on their idle CUs (hgemm.hip).  Element rule (solution/k_nf4.py:40-57):
// byte e / 2 of the packed section, high nibble for even e; absmax = fp32(fp32(code2[qabs[e / 64]]
// * scale2[e / 16384]) + offset2[e / 16384]); out[e] = fp16(fp32(NF4[nibble] * absmax)).
#pragma once
#include "dk_common.h"

// The 16 NF4 values in LDS: every lane of a wave looks up one of the same 16 entries, so the
// reads broadcast instead of conflicting (measured faster on MI355X than a 256-entry table of
// value pairs, whose random 8-byte reads conflict).
__device__ __forceinline__ void dk_fill_lut(float* lut, const float* nf4, int tid) {
  if (tid < 16) lut[tid] = nf4[tid];
}

// Four packed bytes (8 weights) of one first-level block with absmax a -> 8 fp16 as one 16-byte
// vector: fp16(fp32(NF4[nibble] * a)) per weight, the even element in the high nibble.
__device__ __forceinline__ u32x4 dk_dequant_word(uint32_t w, float a, const float* lut) {
  u32x4 o;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t byte = (w >> (8 * b)) & 0xffu;
    o[b] = dk_pack2(dk_h(__fmul_rn(lut[byte >> 4], a)), dk_h(__fmul_rn(lut[byte & 15u], a)));
  }
  return o;
}

namespace dk {

// Dequant work of one GEMM launch: second-level blocks [sb0, sb1) of a repacked layer (section
// pointers of the whole layer), weight e to out[e].
struct SideDequant {
  const u32x4* packed;
  const uint8_t* qabs;
  const float* scale2;
  const float* offset2;
  const float* code2;
  const float* nf4;
  u32x4* out;
  int64_t sb0, sb1;
  int wgs;
};

// The part of a SideDequant that workgroup `id` of its `wgs` runs: a contiguous run of
// second-level blocks (16384 weights, 512 quads of 32), one quad per thread of a 512-thread
// workgroup.  Blocks go in batches of kSideBatch; the loads of the next batch are issued before
// the current one is converted, so their latency overlaps the conversion.  Each wave stages its
// lanes' 64 output bytes in LDS and writes them back lane-contiguous (1 KiB per store
// instruction); loads and stores are non-temporal, so the stream does not displace the GEMM's
// operand lines in L2.  `lds` needs side_dequant_lds bytes, 16-byte aligned.
constexpr int kSideThreads = 512;
constexpr int kSideBatch = 2;
constexpr int kSideStageChunks = 64 * 4 + 4;   // per wave: 64 lanes x 4 chunks, 1 pad per 64
constexpr int side_dequant_lds = 1088 + (kSideThreads / 64) * kSideStageChunks * 16;

struct SideLoads {
  u32x4 w[kSideBatch];
  uint32_t qa[kSideBatch];
  float s2[kSideBatch], o2[kSideBatch];
};

__device__ __forceinline__ void side_load(const SideDequant& s, int64_t b0, int64_t hi, int tid,
                                          SideLoads& L) {
#pragma unroll
  for (int u = 0; u < kSideBatch; ++u) {
    const int64_t sb = b0 + u < hi ? b0 + u : hi - 1;   // past the run: loaded, not stored
    const int64_t quad = sb * kSideThreads + tid;
    L.w[u] = __builtin_nontemporal_load(s.packed + quad);
    L.qa[u] = s.qabs[quad >> 1];
    L.s2[u] = s.scale2[sb];
    L.o2[u] = s.offset2[sb];
  }
}

__device__ __forceinline__ void side_dequant(const SideDequant& s, int id, uint8_t* lds) {
  float* lut = reinterpret_cast<float*>(lds);              // the 16 NF4 values
  float* c2 = reinterpret_cast<float*>(lds + 64);          // the 256 code2 values
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  u32x4* stage = reinterpret_cast<u32x4*>(lds + 1088) + wave * kSideStageChunks;
  dk_fill_lut(lut, s.nf4, tid);
  if (tid < 256) c2[tid] = s.code2[tid];
  const int64_t n = s.sb1 - s.sb0;
  const int64_t lo = s.sb0 + n * id / s.wgs, hi = s.sb0 + n * (id + 1) / s.wgs;
  SideLoads cur, nxt;
  if (lo < hi) side_load(s, lo, hi, tid, cur);
  __syncthreads();   // tables
  for (int64_t b0 = lo; b0 < hi; b0 += kSideBatch) {
    if (b0 + kSideBatch < hi) side_load(s, b0 + kSideBatch, hi, tid, nxt);
#pragma unroll
    for (int u = 0; u < kSideBatch; ++u) {
      if (b0 + u >= hi) break;
      const float amax = dk_absmax(c2[cur.qa[u]], cur.s2[u], cur.o2[u]);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int idx = lane * 4 + j;
        stage[idx + (idx >> 6)] = dk_dequant_word(cur.w[u][j], amax, lut);
      }
      __builtin_amdgcn_wave_barrier();
      u32x4* dst = s.out + (b0 + u) * 2048 + wave * 256;   // 2048 chunks of 8 weights per block
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int idx = j * 64 + lane;
        __builtin_nontemporal_store(stage[idx + (idx >> 6)], dst + idx);
      }
      __builtin_amdgcn_wave_barrier();
    }
    cur = nxt;
  }
}

}  // namespace dk
