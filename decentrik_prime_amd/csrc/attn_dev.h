#pragma once
// Shared device code of the attention kernels (attn_fwd.hip, attn.hip): the QKV layout, the
// block table, the LDS tile layout and DMA, the MFMA and transposing-read helpers.
//
// Variable-length causal GQA attention of the packed batch on gfx950: forward (online softmax) and
// backward (delta, dK/dV per query head, dQ).  Replaces solution/k_attn.py:40-245.
//
// Layout (the fused QKV buffer the QKV epilogue writes): row t of qkv [N, (NQ + 2 NKV) HD] fp16
// holds token t's query heads, then its key heads, then its value heads; query head h reads key /
// value head h / (NQ / NKV).  cu_seqlens [n_seq + 1] delimits the sequences; a block table of
// (sequence, first row) pairs names the workgroups, whose rows never straddle two sequences, so
// the mask is `key <= query` inside a sequence.  Scores are scaled by qk_scale = log2(e) / sqrt(HD)
// and the softmax runs in the exp2 domain; lse [NQ, N] holds m + log2(l) per (head, token).
//
// MFMA orientation: every product is v_mfma_f32_32x32x16_f16, arranged so that the index a
// softmax statistic belongs to sits on the lane.  Forward and dQ compute S^T = K Q^T (keys x
// queries: lane l % 32 is the query, the running max, sum and rescale are per lane) and O^T = V^T
// P^T, taking P^T straight from the score registers: the 32x32 result register v of lane l is row
// 8 (v / 4) + 4 (l / 32) + v % 4, so registers 8 t' .. 8 t' + 7 of a lane hold keys
// 16 t' + 8 (j / 4) + 4 (l / 32) + j % 4 (j = 0..7), and the other operand supplies the same keys
// in the same order, read as columns of the row-major LDS tile by ds_read_b64_tr_b16 (the k order
// of a product is free as long as both operands agree).  dK/dV compute S = Q K^T (the key on the
// lane) and use P and dS the same way.
#include "dk_common.h"

namespace {

constexpr int kHD = 128;          // head size (Qwen2.5: 128)
constexpr int kAThreads = 256;    // 4 waves, 32 query rows (or keys) each
constexpr int kBM = 128;          // queries per forward / dQ workgroup, keys per dK/dV workgroup
constexpr int kBN = 64;           // keys per forward / dQ tile, queries per dK/dV tile
static_assert(kBM == 32 * (kAThreads / 64), "a wave owns 32 rows");

struct AttnArgs {
  const f16* qkv;
  const int32_t* cu;
  const int32_t* tab;
  int n_seq;
  int64_t n_tokens;
  int nq, nkv;
  float qk_scale, sm_scale;
};

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int v = 0; v < 16; ++v) z[v] = 0.0f;
  return z;
}

__device__ __forceinline__ f16x8 zero8() {
  f16x8 z;
#pragma unroll
  for (int e = 0; e < 8; ++e) z[e] = (f16)0.0f;
  return z;
}

__device__ __forceinline__ f32x16 mfma(const f16x8& a, const f16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f16x4 read_tr(const f16* q) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(q)));
}

// K / V (or Q / dO) tiles in a ring of LDS stages filled by LDS DMA (global_load_lds_dwordx4:
// no registers, the next tiles' loads in flight while this one is computed on).  A tile is kBN
// rows of 256 bytes with no padding; the 16-byte chunks of row r are permuted by swz16(r), so
// that both reads of the tile are free of bank conflicts: the S^T operand (16 consecutive rows,
// one chunk each) and the transposing V reads (4 rows x 2 adjacent chunks per 16-lane group).
constexpr int kFwdStages = 4;                 // tiles t, t + 1 in use, t + 2, t + 3 in flight
constexpr int kTileHalves = kBN * kHD;        // one operand of one stage: 16 KB

__device__ __forceinline__ int swz16(int r) {
  return ((r & 3) << 1) | ((r >> 2) & 1) | (((r >> 3) & 1) << 3);
}
// offset (halves) of column c of row r in a swizzled tile
__device__ __forceinline__ int sw_off(int r, int c) {
  return r * kHD + ((((c >> 3) ^ swz16(r))) << 3) + (c & 7);
}

__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(size_t)(__attribute__((address_space(3))) const void*)p;
}

// 16 bytes per lane from global memory into LDS at lds + 16 * lane (inline assembly, so that the
// compiler does not put a wait for it before every LDS read: the kernel counts these loads with
// its own vmcnt waits; M0, the LDS address, is saved and restored around it).
__device__ __forceinline__ void dma16(const void* src, unsigned lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(src)
      : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Column (col + l % 32) of rows p .. p + 3 and p + 8 .. p + 11 of a swizzled tile, the 8 values of
// MFMA k index j = 0..7 for a lane half whose p = 16 t + 4 (l / 32).  ds_read_b64_tr_b16: within
// a 16-lane group, lane 4a + b receives element b of the 4-half pieces addressed by lanes a,
// a + 4, a + 8, a + 12; lane x addresses row p + x / 4 at columns col + 16 (group) + 4 (x % 4),
// so lane x' of the group receives column col + 16 (group) + x' of the four rows.
__device__ __forceinline__ f16x8 read_col8_sw(const f16* tile, int p, int col) {
  const int lane = threadIdx.x & 63;
  const int r = p + ((lane & 15) >> 2), c = col + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
  const f16x4 lo = read_tr(tile + sw_off(r, c)), hi = read_tr(tile + sw_off(r + 8, c));
  return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// 2^x on the hardware exponential (v_exp_f32); arguments here are <= 0 (scores minus their row
// maximum or log-sum-exp), results below the normal range flush to zero.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// The sequence of a block-table entry; false when the entry names no sequence, a sequence that
// does not lie within the n_tokens rows, or a block start at or past the sequence's end (an empty
// sequence included).  A workgroup whose entry is refused returns before any load, so every row
// a kernel reads unconditionally (row start of the sequence) exists whatever the tables hold.
__device__ __forceinline__ bool block_of(const AttnArgs& a, int blk, int64_t* s0, int* seqlen,
                                         int* start) {
  const int seq = a.tab[2 * blk];
  *start = a.tab[2 * blk + 1];
  if (seq < 0 || seq >= a.n_seq || *start < 0) return false;
  *s0 = a.cu[seq];
  *seqlen = a.cu[seq + 1] - a.cu[seq];
  return *s0 >= 0 && *seqlen > 0 && *start < *seqlen && *s0 + *seqlen <= a.n_tokens;
}

// the launch arguments, with the checks every attention entry point shares
inline int attn_args(AttnArgs& a, const void* qkv, const int32_t* cu, int32_t n_seq,
                     const int32_t* tab, int32_t n_blocks, int64_t n_tokens, int32_t nq,
                     int32_t nkv, int32_t hd) {
  if (hd != kHD || nq < 1 || nkv < 1 || nq % nkv || nq > 65535 || n_seq < 0 || n_blocks < 0 ||
      n_tokens < 0)
    return DK_ERR_INVALID;
  if (n_blocks > 0 && (!qkv || !cu || !tab || n_seq < 1)) return DK_ERR_INVALID;
  if (!dk_aligned(qkv, 16) || !dk_aligned(cu, 4) || !dk_aligned(tab, 4)) return DK_ERR_ALIGN;
  const double log2e = 1.4426950408889634;
  a = AttnArgs{(const f16*)qkv, cu, tab, n_seq, n_tokens, nq, nkv,
               (float)(log2e / __builtin_sqrt((double)hd)), (float)(1.0 / __builtin_sqrt((double)hd))};
  return 0;
}

}  // namespace
