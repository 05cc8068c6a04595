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

// One wave's share of a dequant: 64 lanes x kWaveDwords packed dwords (8 weights each) from dword
// d_wave on, dword j of lane l at d_wave + 64 j + l, inside one second-level block (2048 dwords),
// so scale2/offset2 are wave-uniform.  The wave spans 8 kWaveDwords first-level blocks: lane k
// loads the codes of blocks k, k + 64, ... and forms their absmax once, and each dword takes its
// block's absmax from the owning lane by a cross-lane read.  Every load goes out in
// dq_wave_load, before any conversion; dq_wave_store converts and writes each dword's 8 fp16 as
// one 16-byte store (the wave's store instruction writes 1 KiB contiguous).  Dwords past `last`
// are loaded at clamped addresses and not stored.
constexpr int kWaveDwords = 32;
constexpr int kWaveOwn = kWaveDwords / 8;   // first-level codes per lane
static_assert(64 * kWaveDwords <= DK_ELEMS_PER_SB / 8, "a wave within one second-level block");

struct WaveLoads {
  uint32_t w[kWaveDwords];
  uint8_t q[kWaveOwn];
  float s2, o2;
};

__device__ __forceinline__ void dq_wave_load(const uint32_t* __restrict__ packed,
                                             const uint8_t* __restrict__ qabs,
                                             const float* __restrict__ scale2,
                                             const float* __restrict__ offset2, int64_t d_wave,
                                             int64_t last, int lane, WaveLoads& L) {
  const int64_t blk_last = last / 8;
#pragma unroll
  for (int o = 0; o < kWaveOwn; ++o) {
    const int64_t blk = d_wave / 8 + 64 * o + lane;
    L.q[o] = qabs[blk < blk_last ? blk : blk_last];
  }
  const int64_t sb = (d_wave < last ? d_wave : last) / (DK_ELEMS_PER_SB / 8);
  L.s2 = scale2[sb];
  L.o2 = offset2[sb];
#pragma unroll
  for (int j = 0; j < kWaveDwords; ++j) {
    const int64_t d = d_wave + 64 * j + lane;
    L.w[j] = __builtin_nontemporal_load(packed + (d < last ? d : last));
  }
}

// c2, lut: the 256-entry code table and the 16 NF4 values in LDS.  nt: non-temporal stores.
template <bool NT>
__device__ __forceinline__ void dq_wave_store(const WaveLoads& L, const float* c2, const float* lut,
                                              u32x4* __restrict__ out, int64_t d_wave,
                                              int64_t last, int lane) {
  float amax_own[kWaveOwn];
#pragma unroll
  for (int o = 0; o < kWaveOwn; ++o) amax_own[o] = dk_absmax(c2[L.q[o]], L.s2, L.o2);
#pragma unroll
  for (int j = 0; j < kWaveDwords; ++j) {
    // dword j of lane l is in block 8 j + l / 8 of the wave: lane (8 j + l / 8) % 64, entry 8 j / 64
    const float amax = __shfl(amax_own[j / 8], 8 * (j % 8) + (lane >> 3));
    const int64_t d = d_wave + 64 * j + lane;
    const u32x4 o = dk_dequant_word(L.w[j], amax, lut);
    if (d <= last) {
      if (NT) __builtin_nontemporal_store(o, out + d);
      else out[d] = o;
    }
  }
}

// The part of a SideDequant that workgroup `id` of its `wgs` runs (512 threads, 8 waves): the
// second-level blocks sb0 + g, sb0 + g + 8 wgs, ... for its wave g = 8 id + w, one block per wave
// at a time, the next block's loads issued before the current one is converted.  Stores are
// non-temporal, so the stream does not displace the GEMM's operand lines in L2.  `lds` needs
// side_dequant_lds bytes.
constexpr int kSideThreads = 512;
constexpr int side_dequant_lds = 64 + 1024;

__device__ __forceinline__ void side_dequant(const SideDequant& s, int id, uint8_t* lds) {
  float* lut = reinterpret_cast<float*>(lds);              // the 16 NF4 values
  float* c2 = reinterpret_cast<float*>(lds + 64);          // the 256 code2 values
  const int tid = threadIdx.x, lane = tid & 63;
  const int g = id * (kSideThreads / 64) + __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t stride = (int64_t)s.wgs * (kSideThreads / 64);
  const uint32_t* packed = reinterpret_cast<const uint32_t*>(s.packed);
  const int64_t last = s.sb1 * (DK_ELEMS_PER_SB / 8) - 1;   // the run's last dword
  const float c2v = s.code2[tid & 255], lutv = s.nf4[tid & 15];
  WaveLoads cur, nxt;
  int64_t sb = s.sb0 + g;
  if (sb < s.sb1) dq_wave_load(packed, s.qabs, s.scale2, s.offset2, sb * 2048, last, lane, cur);
  if (tid < 256) c2[tid] = c2v;
  if (tid < 16) lut[tid] = lutv;
  __syncthreads();   // tables
  for (; sb < s.sb1; sb += stride) {
    if (sb + stride < s.sb1)
      dq_wave_load(packed, s.qabs, s.scale2, s.offset2, (sb + stride) * 2048, last, lane, nxt);
    dq_wave_store<true>(cur, c2, lut, s.out, sb * 2048, last, lane);
    cur = nxt;
  }
}

}  // namespace dk
