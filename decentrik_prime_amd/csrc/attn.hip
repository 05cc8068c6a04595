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
// of a product is free as long as both operands agree).  dK/dV compute S = Q K^T (the key on the lane) and use P and dS the same way.
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

// The sequence of a block-table entry; false when the entry names no sequence or a sequence that
// does not lie within the n_tokens rows (then every row and loop of the workgroup stays in bounds
// whatever the tables hold).
__device__ __forceinline__ bool block_of(const AttnArgs& a, int blk, int64_t* s0, int* seqlen,
                                         int* start) {
  const int seq = a.tab[2 * blk];
  *start = a.tab[2 * blk + 1];
  if (seq < 0 || seq >= a.n_seq || *start < 0) return false;
  *s0 = a.cu[seq];
  *seqlen = a.cu[seq + 1] - a.cu[seq];
  return *s0 >= 0 && *seqlen >= 0 && *s0 + *seqlen <= a.n_tokens;
}

// forward (solution/k_attn.py:40-83): one workgroup per (block of kBM queries, query head)
__global__ __launch_bounds__(kAThreads) void attn_fwd_kernel(AttnArgs a, f16* __restrict__ out,
                                                             float* __restrict__ lse) {
  int64_t s0;
  int seqlen, mstart;
  if (!block_of(a, blockIdx.x, &s0, &seqlen, &mstart)) return;
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(w);
  const int64_t ROW = (int64_t)(a.nq + 2 * a.nkv) * kHD;
  const int kvh = h / (a.nq / a.nkv);
  const int m = mstart + 32 * w + c;
  const bool mval = m < seqlen && s0 + m < a.n_tokens;
  __shared__ __attribute__((aligned(1024))) f16 Ks[kFwdStages * kTileHalves];
  __shared__ __attribute__((aligned(1024))) f16 Vs[kFwdStages * kTileHalves];

  f32x16 oacc[kHD / 32];
#pragma unroll
  for (int hb = 0; hb < kHD / 32; ++hb) oacc[hb] = zero16();
  float m_i = -1.0e30f, l_i = 0.0f;
  const int hi = mstart + kBM < seqlen ? mstart + kBM : seqlen;
  const int n_tiles = (hi + kBN - 1) / kBN;
  const f16* kbase = a.qkv + s0 * ROW + (int64_t)(a.nq + kvh) * kHD;
  const f16* vbase = a.qkv + s0 * ROW + (int64_t)(a.nq + a.nkv + kvh) * kHD;
  // tile t into stage st: instruction i of wave w fills the stage's chunks (4 i + w) 64 + lane,
  // row q / 16 (rows past the sequence read its last row: finite, and masked to p = 0)
  constexpr int kLoads = kTileHalves / 8 / kAThreads;   // per operand per lane: 4
  auto issue = [&](int t, int st) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int q = (4 * i + wave) * 64 + lane, r = q >> 4;
      const int row = t * kBN + r < seqlen ? t * kBN + r : seqlen - 1;
      const int64_t src = (int64_t)row * ROW + (((q & 15) ^ swz16(r)) << 3);
      const int dst = st * kTileHalves + (4 * i + wave) * 512;
      dma16(kbase + src, __builtin_amdgcn_readfirstlane(lds_addr(Ks + dst)));
      dma16(vbase + src, __builtin_amdgcn_readfirstlane(lds_addr(Vs + dst)));
    }
  };
  issue(0, 0);
  if (n_tiles > 1) issue(1, 1);
  if (n_tiles > 2) issue(2, 2);
  // this lane's query row as the B operand (rows past the sequence: zeros).  Loaded at a clamped
  // row unconditionally and selected at once, so the compiler's wait for these loads stands here
  // (it then also covers the tiles issued above) and not inside the loop, where it would wait for
  // the tiles in flight every iteration.
  f16x8 qf[kHD / 16];
  {
    const f16* qrow = a.qkv + (s0 + (mval ? m : mstart)) * ROW + h * kHD + 8 * hl;
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) qf[s] = *reinterpret_cast<const f16x8*>(qrow + 16 * s);
    // (the empty asm needs the loaded values: the compiler can neither predicate the loads on
    // mval nor defer their wait into the loop)
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) asm volatile("" : "+v"(qf[s]));
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) qf[s] = mval ? qf[s] : zero8();
  }
  // S^T = K Q^T of the tile in stage st: keys kb * 32 + (row of the result), queries on the lanes
  auto scores = [&](f32x16 (&acc)[2], int st) {
    const f16* Kt = Ks + st * kTileHalves;
    acc[0] = acc[1] = zero16();
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        acc[kb] = mfma(*reinterpret_cast<const f16x8*>(Kt + sw_off(kb * 32 + c, 16 * s + 8 * hl)),
                       qf[s], acc[kb]);
  };
  // software pipeline: iteration t runs the score MFMAs of tile t + 1 beside the softmax of tile
  // t (its VALU work), then O += V_t P_t.  Tiles t and t + 1 are in LDS at its start.
  if (n_tiles > 2) wait_vmem<2 * kLoads>();
  else wait_vmem<0>();
  __syncthreads();
  f32x16 sc[2];
  scores(sc, 0);
  for (int t = 0; t < n_tiles; ++t) {
    // stage (t + 3) % 4 held tile t - 1, whose last reader (O += V P of iteration t - 1) every wave
    // finished before the barrier that ended that iteration
    if (t + 3 < n_tiles) issue(t + 3, (t + 3) % kFwdStages);
    const f16* Vt = Vs + (t % kFwdStages) * kTileHalves;
    const int n0 = t * kBN;
    // tile t + 1's scores (past the last tile: a stale stage, never used)
    f32x16 sn[2];
    scores(sn, (t + 1) % kFwdStages);
    // softmax of tile t in the exp2 domain: the row maximum of the raw scores, scaled once (the
    // scaling is monotonic, so this is the maximum of the scaled scores), and
    // p = 2^(s * qk_scale - m) with one rounding
    float mx = -1.0e30f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int n = n0 + kb * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
        const float sv = n <= m && n < seqlen ? sc[kb][v] : -1.0e30f;
        sc[kb][v] = sv;
        mx = fmaxf(mx, sv);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_i, __fmul_rn(mx, a.qk_scale));
    const float alpha = ex2(__fsub_rn(m_i, m_new));
    float rs = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = ex2(__builtin_fmaf(sc[kb][v], a.qk_scale, -m_new));
        sc[kb][v] = p;
        rs = __fadd_rn(rs, p);
      }
    rs = __fadd_rn(rs, __shfl_xor(rs, 32));
    l_i = __fadd_rn(__fmul_rn(l_i, alpha), rs);
    m_i = m_new;
#pragma unroll
    for (int hb = 0; hb < kHD / 32; ++hb)
#pragma unroll
      for (int v = 0; v < 16; ++v) oacc[hb][v] = __fmul_rn(oacc[hb][v], alpha);
    // the 16 score MFMAs of tile t + 1 spread among the softmax's VALU work
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // an operand read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // an MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);   // VALU
    }
    // O^T += V^T P^T over the tile's 64 keys, 16 per step
#pragma unroll
    for (int tt = 0; tt < kBN / 16; ++tt) {
      const int kb = tt >> 1, i0 = 8 * (tt & 1);
      f16x8 pf;
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[j] = (f16)sc[kb][i0 + j];
#pragma unroll
      for (int hb = 0; hb < kHD / 32; ++hb)
        oacc[hb] = mfma(read_col8_sw(Vt, 16 * tt + 4 * hl, hb * 32), pf, oacc[hb]);
    }
    // tile t + 2 landed (tile t + 3 may still be in flight) and visible to every wave, and every
    // wave is done with stage t % 4
    if (t + 3 < n_tiles) wait_vmem<2 * kLoads>();
    else wait_vmem<0>();
    __syncthreads();
    sc[0] = sn[0];
    sc[1] = sn[1];
  }
  if (!mval) return;
  // result register v of block hb: head column hb * 32 + 8 (v / 4) + 4 (l / 32) + v % 4
  f16* orow = out + (s0 + m) * (int64_t)(a.nq * kHD) + h * kHD;
#pragma unroll
  for (int hb = 0; hb < kHD / 32; ++hb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (f16)__fdiv_rn(oacc[hb][4 * g + e], l_i);
      *reinterpret_cast<f16x4*>(orow + hb * 32 + 8 * g + 4 * hl) = o;
    }
  if (hl == 0) lse[(int64_t)h * a.n_tokens + s0 + m] = __fadd_rn(m_i, log2f(l_i));
}

// delta[h][t] = sum_d O[t][h][d] dO[t][h][d] (solution/k_attn.py:84-94): 16 lanes per (token, head)
__global__ __launch_bounds__(kAThreads) void attn_delta_kernel(const f16* __restrict__ o,
                                                               const f16* __restrict__ dout,
                                                               float* __restrict__ delta,
                                                               int64_t n_tokens, int nq) {
  const int64_t pair = (int64_t)blockIdx.x * (kAThreads / 16) + (threadIdx.x >> 4);
  if (pair >= n_tokens * nq) return;
  const int64_t t = pair / nq;
  const int hh = (int)(pair % nq), e = (threadIdx.x & 15) * 8;
  const int64_t off = t * nq * kHD + hh * kHD + e;
  const f16x8 ov = *reinterpret_cast<const f16x8*>(o + off);
  const f16x8 gv = *reinterpret_cast<const f16x8*>(dout + off);
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) s = __fadd_rn(s, __fmul_rn((float)ov[j], (float)gv[j]));
#pragma unroll
  for (int x = 1; x < 16; x <<= 1) s = __fadd_rn(s, __shfl_xor(s, x));
  if ((threadIdx.x & 15) == 0) delta[(int64_t)hh * n_tokens + t] = s;
}

// dQ (solution/k_attn.py:142-182): one workgroup per (block of kBM queries, query head), key
// tiles of kBN up to the diagonal, in the forward's four-stage K/V ring; the S^T and dP^T MFMAs of
// tile t + 1 run beside the dS work of tile t
__global__ __launch_bounds__(kAThreads) void attn_dq_kernel(AttnArgs a, const f16* __restrict__ dout,
                                                            const float* __restrict__ lse,
                                                            const float* __restrict__ delta,
                                                            float* __restrict__ dq) {
  int64_t s0;
  int seqlen, mstart;
  if (!block_of(a, blockIdx.x, &s0, &seqlen, &mstart)) return;
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(w);
  const int64_t ROW = (int64_t)(a.nq + 2 * a.nkv) * kHD, OROW = (int64_t)a.nq * kHD;
  const int kvh = h / (a.nq / a.nkv);
  const int m = mstart + 32 * w + c;
  const bool mval = m < seqlen && s0 + m < a.n_tokens;
  __shared__ __attribute__((aligned(1024))) f16 Ks[kFwdStages * kTileHalves];
  __shared__ __attribute__((aligned(1024))) f16 Vs[kFwdStages * kTileHalves];

  const int hi = mstart + kBM < seqlen ? mstart + kBM : seqlen;
  const int n_tiles = (hi + kBN - 1) / kBN;
  const f16* kbase = a.qkv + s0 * ROW + (int64_t)(a.nq + kvh) * kHD;
  const f16* vbase = a.qkv + s0 * ROW + (int64_t)(a.nq + a.nkv + kvh) * kHD;
  constexpr int kLoads = kTileHalves / 8 / kAThreads;
  auto issue = [&](int t, int st) {
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int q = (4 * i + wave) * 64 + lane, r = q >> 4;
      const int row = t * kBN + r < seqlen ? t * kBN + r : seqlen - 1;
      const int64_t src = (int64_t)row * ROW + (((q & 15) ^ swz16(r)) << 3);
      const int dst = st * kTileHalves + (4 * i + wave) * 512;
      dma16(kbase + src, __builtin_amdgcn_readfirstlane(lds_addr(Ks + dst)));
      dma16(vbase + src, __builtin_amdgcn_readfirstlane(lds_addr(Vs + dst)));
    }
  };
  issue(0, 0);
  if (n_tiles > 1) issue(1, 1);
  if (n_tiles > 2) issue(2, 2);
  // this lane's query and dO rows and statistics, loaded at a clamped row and selected at once
  // (the compiler's wait for them stands here, not in the loop)
  f16x8 qf[kHD / 16], dof[kHD / 16];
  float lse_m, dl_m;
  {
    const int64_t rr = s0 + (mval ? m : mstart);
    const f16* qrow = a.qkv + rr * ROW + h * kHD + 8 * hl;
    const f16* drow = dout + rr * OROW + h * kHD + 8 * hl;
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) {
      qf[s] = *reinterpret_cast<const f16x8*>(qrow + 16 * s);
      dof[s] = *reinterpret_cast<const f16x8*>(drow + 16 * s);
    }
    lse_m = lse[(int64_t)h * a.n_tokens + rr];
    dl_m = delta[(int64_t)h * a.n_tokens + rr];
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) asm volatile("" : "+v"(qf[s]), "+v"(dof[s]));
    asm volatile("" : "+v"(lse_m), "+v"(dl_m));
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) {
      qf[s] = mval ? qf[s] : zero8();
      dof[s] = mval ? dof[s] : zero8();
    }
    lse_m = mval ? lse_m : 0.0f;
    dl_m = mval ? dl_m : 0.0f;
  }
  f32x16 dqacc[kHD / 32];
#pragma unroll
  for (int hb = 0; hb < kHD / 32; ++hb) dqacc[hb] = zero16();
  // S^T = K Q^T and dP^T = V dO^T of the tile in stage st: keys kb * 32 + (row), queries on lanes
  auto products = [&](f32x16 (&sacc)[2], f32x16 (&dpacc)[2], int st) {
    const f16* Kt = Ks + st * kTileHalves;
    const f16* Vt = Vs + st * kTileHalves;
    sacc[0] = sacc[1] = dpacc[0] = dpacc[1] = zero16();
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const int o = sw_off(kb * 32 + c, 16 * s + 8 * hl);
        sacc[kb] = mfma(*reinterpret_cast<const f16x8*>(Kt + o), qf[s], sacc[kb]);
        dpacc[kb] = mfma(*reinterpret_cast<const f16x8*>(Vt + o), dof[s], dpacc[kb]);
      }
  };
  if (n_tiles > 2) wait_vmem<2 * kLoads>();
  else wait_vmem<0>();
  __syncthreads();
  f32x16 sc[2], dc[2];
  products(sc, dc, 0);
  for (int t = 0; t < n_tiles; ++t) {
    if (t + 3 < n_tiles) issue(t + 3, (t + 3) % kFwdStages);
    const f16* Kt = Ks + (t % kFwdStages) * kTileHalves;
    const int n0 = t * kBN;
    f32x16 sn[2], dn[2];
    products(sn, dn, (t + 1) % kFwdStages);
    const bool full = n0 + kBN - 1 <= mstart + 32 * w && n0 + kBN <= seqlen;
    // computed for every score and then selected (a conditional exponential becomes a branch)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int n = n0 + kb * 32 + 8 * (v >> 2) + 4 * hl + (v & 3);
        const float e = ex2(__fsub_rn(__fmul_rn(sc[kb][v], a.qk_scale), lse_m));
        const bool keep = mval & (full | ((n <= m) & (n < seqlen)));   // no short-circuit
        const float p = keep ? e : 0.0f;
        sc[kb][v] = __fmul_rn(p, __fsub_rn(dc[kb][v], dl_m));   // dS^T
      }
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // an operand read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // an MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // VALU
    }
    // dQ^T += K^T dS^T
#pragma unroll
    for (int tt = 0; tt < kBN / 16; ++tt) {
      const int kb = tt >> 1, i0 = 8 * (tt & 1);
      f16x8 dsf;
#pragma unroll
      for (int j = 0; j < 8; ++j) dsf[j] = (f16)sc[kb][i0 + j];
#pragma unroll
      for (int hb = 0; hb < kHD / 32; ++hb)
        dqacc[hb] = mfma(read_col8_sw(Kt, 16 * tt + 4 * hl, hb * 32), dsf, dqacc[hb]);
    }
    if (t + 3 < n_tiles) wait_vmem<2 * kLoads>();
    else wait_vmem<0>();
    __syncthreads();
    sc[0] = sn[0];
    sc[1] = sn[1];
    dc[0] = dn[0];
    dc[1] = dn[1];
  }
  if (!mval) return;
  float* qrow = dq + (s0 + m) * OROW + h * kHD;
#pragma unroll
  for (int hb = 0; hb < kHD / 32; ++hb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = __fmul_rn(dqacc[hb][4 * g + e], a.sm_scale);
      *reinterpret_cast<f32x4*>(qrow + hb * 32 + 8 * g + 4 * hl) = o;
    }
}

// 4 bytes per lane from global memory into LDS at lds + 4 * lane (the dword form of dma16).
__device__ __forceinline__ void dma4(const void* src, unsigned lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dword %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(src)
      : "memory");
}

// dK, dV per query head (solution/k_attn.py:97-139): one workgroup per (block of kBM keys, query
// head), query tiles of kBN from the block's first key to the end of the sequence; fp32 partials
// [N, NQ HD] that the QKV epilogue backward sums over each group of NQ / NKV heads.  The Q and dO
// tiles and the tiles' lse and delta rows come through a four-stage LDS ring filled by LDS DMA
// (swizzled rows as in the forward; the statistics by dword DMA, one lane per query, waves 0
// and 1), and the S and dP MFMAs of tile t + 1 run beside the P / dS work of tile t.
constexpr int kBwdStages = 4;

__global__ __launch_bounds__(kAThreads) void attn_dkdv_kernel(AttnArgs a, const f16* __restrict__ dout,
                                                              const float* __restrict__ lse,
                                                              const float* __restrict__ delta,
                                                              float* __restrict__ dkp,
                                                              float* __restrict__ dvp) {
  int64_t s0;
  int seqlen, nstart;
  if (!block_of(a, blockIdx.x, &s0, &seqlen, &nstart)) return;
  const int h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hl = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(w);
  const int64_t ROW = (int64_t)(a.nq + 2 * a.nkv) * kHD, OROW = (int64_t)a.nq * kHD;
  const int kvh = h / (a.nq / a.nkv);
  const int n = nstart + 32 * w + c;   // this lane's key
  const bool nval = n < seqlen && s0 + n < a.n_tokens;
  __shared__ __attribute__((aligned(1024))) f16 Qs[kBwdStages * kTileHalves];
  __shared__ __attribute__((aligned(1024))) f16 Ds[kBwdStages * kTileHalves];
  __shared__ __attribute__((aligned(16))) float lse_s[kBwdStages][kBN], dl_s[kBwdStages][kBN];

  const int n_tiles = nstart < seqlen ? (seqlen - nstart + kBN - 1) / kBN : 0;
  const f16* qbase = a.qkv + s0 * ROW + (int64_t)h * kHD;
  const f16* dbase = dout + s0 * OROW + (int64_t)h * kHD;
  constexpr int kLoads = kTileHalves / 8 / kAThreads;   // per operand per lane: 4
  // query tile t (queries nstart + 64 t ...) into stage st; rows past the sequence read its last
  // row (finite, masked to p = 0); wave 0 also fetches the tile's lse, wave 1 its delta
  auto issue = [&](int t, int st) {
    const int m0 = nstart + t * kBN;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int q = (4 * i + wave) * 64 + lane, r = q >> 4;
      const int row = m0 + r < seqlen ? m0 + r : seqlen - 1;
      const int off = ((q & 15) ^ swz16(r)) << 3;
      const int dst = st * kTileHalves + (4 * i + wave) * 512;
      dma16(qbase + (int64_t)row * ROW + off, __builtin_amdgcn_readfirstlane(lds_addr(Qs + dst)));
      dma16(dbase + (int64_t)row * OROW + off, __builtin_amdgcn_readfirstlane(lds_addr(Ds + dst)));
    }
    if (wave < 2) {
      const int qq = m0 + lane < seqlen ? m0 + lane : seqlen - 1;
      const float* src = (wave == 0 ? lse : delta) + (int64_t)h * a.n_tokens + s0 + qq;
      dma4(src, __builtin_amdgcn_readfirstlane(lds_addr(wave == 0 ? lse_s[st] : dl_s[st])));
    }
  };
  // wait until at most `tiles` tiles of this wave's loads are in flight (waves 0 and 1 issue one
  // more load per tile)
  auto wait_tiles = [&](int tiles) {
    if (wave < 2) {
      if (tiles >= 2) wait_vmem<2 * (2 * kLoads + 1)>();
      else if (tiles == 1) wait_vmem<2 * kLoads + 1>();
      else wait_vmem<0>();
    } else {
      if (tiles >= 2) wait_vmem<2 * 2 * kLoads>();
      else if (tiles == 1) wait_vmem<2 * kLoads>();
      else wait_vmem<0>();
    }
  };
  if (n_tiles > 0) issue(0, 0);
  if (n_tiles > 1) issue(1, 1);
  if (n_tiles > 2) issue(2, 2);

  // this lane's key and value rows as B operands, loaded at a clamped row and selected at once
  // (the compiler's wait for them stands here, not in the loop)
  f16x8 kf[kHD / 16], vf[kHD / 16];
  {
    const int64_t rr = s0 + (nval ? n : nstart);
    const f16* krow = a.qkv + rr * ROW + (int64_t)(a.nq + kvh) * kHD + 8 * hl;
    const f16* vrow = a.qkv + rr * ROW + (int64_t)(a.nq + a.nkv + kvh) * kHD + 8 * hl;
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) {
      kf[s] = *reinterpret_cast<const f16x8*>(krow + 16 * s);
      vf[s] = *reinterpret_cast<const f16x8*>(vrow + 16 * s);
    }
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) asm volatile("" : "+v"(kf[s]), "+v"(vf[s]));
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s) {
      kf[s] = nval ? kf[s] : zero8();
      vf[s] = nval ? vf[s] : zero8();
    }
  }
  f32x16 dkacc[kHD / 32], dvacc[kHD / 32];
#pragma unroll
  for (int hb = 0; hb < kHD / 32; ++hb) dkacc[hb] = dvacc[hb] = zero16();
  // S = Q K^T and dP = dO V^T of the tile in stage st: queries qb * 32 + (row of the result),
  // keys on the lanes
  auto products = [&](f32x16 (&sacc)[2], f32x16 (&dpacc)[2], int st) {
    const f16* Qt = Qs + st * kTileHalves;
    const f16* Dt = Ds + st * kTileHalves;
    sacc[0] = sacc[1] = dpacc[0] = dpacc[1] = zero16();
#pragma unroll
    for (int s = 0; s < kHD / 16; ++s)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const int o = sw_off(qb * 32 + c, 16 * s + 8 * hl);
        sacc[qb] = mfma(*reinterpret_cast<const f16x8*>(Qt + o), kf[s], sacc[qb]);
        dpacc[qb] = mfma(*reinterpret_cast<const f16x8*>(Dt + o), vf[s], dpacc[qb]);
      }
  };
  if (n_tiles > 0) {
    wait_tiles(n_tiles > 2 ? 1 : 0);   // tiles 0 and 1 landed
    __syncthreads();
  }
  f32x16 sc[2], dc[2];
  if (n_tiles > 0) products(sc, dc, 0);
  for (int t = 0; t < n_tiles; ++t) {
    // stage (t + 3) % 4 held tile t - 1, whose last reader every wave finished before the
    // barrier that ended iteration t - 1
    if (t + 3 < n_tiles) issue(t + 3, (t + 3) % kBwdStages);
    const int st = t % kBwdStages;
    const int m0 = nstart + t * kBN;
    // tile t + 1's products (past the last tile: a stale stage, never used)
    f32x16 sn[2], dn[2];
    products(sn, dn, (t + 1) % kBwdStages);
    // every query of the tile at or after every key of this wave, all inside the sequence
    const bool full = m0 >= nstart + 32 * w + 31 && m0 + kBN <= seqlen;
    // the statistics of this lane's 32 queries of the tile: rows qb * 32 + 8 g + 4 (l / 32) + 0..3
    f32x4 ls[2][4], ds[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        ls[qb][g] = *reinterpret_cast<const f32x4*>(&lse_s[st][qb * 32 + 8 * g + 4 * hl]);
        ds[qb][g] = *reinterpret_cast<const f32x4*>(&dl_s[st][qb * 32 + 8 * g + 4 * hl]);
      }
    // computed for every score and then selected: a conditional exponential becomes a branch per
    // score
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int r = qb * 32 + 8 * (v >> 2) + 4 * hl + (v & 3), q = m0 + r;
        const float e = ex2(__fsub_rn(__fmul_rn(sc[qb][v], a.qk_scale), ls[qb][v >> 2][v & 3]));
        const bool keep = nval & (full | ((q >= n) & (q < seqlen)));   // no short-circuit
        const float p = keep ? e : 0.0f;
        sc[qb][v] = p;                                                           // P
        dc[qb][v] = __fmul_rn(p, __fsub_rn(dc[qb][v], ds[qb][v >> 2][v & 3]));    // dS
      }
    // the 32 products of tile t + 1 spread among this work
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // an operand read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // an MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // VALU
    }
    // dV += P^T dO, dK += dS^T Q over the tile's 64 queries, 16 per step
    const f16* Qt = Qs + st * kTileHalves;
    const f16* Dt = Ds + st * kTileHalves;
#pragma unroll
    for (int tt = 0; tt < kBN / 16; ++tt) {
      const int qb = tt >> 1, i0 = 8 * (tt & 1);
      f16x8 pf, dsf;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        pf[j] = (f16)sc[qb][i0 + j];
        dsf[j] = (f16)dc[qb][i0 + j];
      }
#pragma unroll
      for (int hb = 0; hb < kHD / 32; ++hb) {
        dvacc[hb] = mfma(pf, read_col8_sw(Dt, 16 * tt + 4 * hl, hb * 32), dvacc[hb]);
        dkacc[hb] = mfma(dsf, read_col8_sw(Qt, 16 * tt + 4 * hl, hb * 32), dkacc[hb]);
      }
    }
    // tile t + 2 landed and visible to every wave, every wave done with stage t % 4
    wait_tiles(t + 3 < n_tiles ? 1 : 0);
    __syncthreads();
    sc[0] = sn[0];
    sc[1] = sn[1];
    dc[0] = dn[0];
    dc[1] = dn[1];
  }
  // result register v of block hb: key 32 w + 8 (v / 4) + 4 (l / 32) + v % 4, column hb * 32 + c
#pragma unroll
  for (int v = 0; v < 16; ++v) {
    const int key = nstart + 32 * w + 8 * (v >> 2) + 4 * hl + (v & 3);
    if (key >= seqlen || s0 + key >= a.n_tokens) continue;
    const int64_t off = (s0 + key) * OROW + h * kHD + c;
#pragma unroll
    for (int hb = 0; hb < kHD / 32; ++hb) {
      dkp[off + hb * 32] = __fmul_rn(dkacc[hb][v], a.sm_scale);
      dvp[off + hb * 32] = dvacc[hb][v];
    }
  }
}

int attn_args(AttnArgs& a, const void* qkv, const int32_t* cu, int32_t n_seq, const int32_t* tab,
              int32_t n_blocks, int64_t n_tokens, int32_t nq, int32_t nkv, int32_t hd) {
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

extern "C" int dk_attn_fwd(const void* qkv, const int32_t* cu_seqlens, int32_t n_seq,
                           const int32_t* block_table, int32_t n_blocks, int64_t n_tokens,
                           int32_t nq, int32_t nkv, int32_t hd, void* out, float* lse,
                           hipStream_t stream) {
  AttnArgs a;
  if (int e = attn_args(a, qkv, cu_seqlens, n_seq, block_table, n_blocks, n_tokens, nq, nkv, hd))
    return e;
  if (n_blocks == 0) return 0;
  if (!out || !lse) return DK_ERR_INVALID;
  if (!dk_aligned(out, 16) || !dk_aligned(lse, 4)) return DK_ERR_ALIGN;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)n_blocks, (unsigned)nq), dim3(kAThreads), 0,
                     stream, a, (f16*)out, lse);
  DK_CHECK_LAUNCH();
  return 0;
}

extern "C" int dk_attn_bwd(const void* qkv, const void* out, const float* lse, const void* dout,
                           const int32_t* cu_seqlens, int32_t n_seq, const int32_t* block_table,
                           int32_t n_blocks, int64_t n_tokens, int32_t nq, int32_t nkv, int32_t hd,
                           float* delta, float* dq, float* dkp, float* dvp, hipStream_t stream) {
  AttnArgs a;
  if (int e = attn_args(a, qkv, cu_seqlens, n_seq, block_table, n_blocks, n_tokens, nq, nkv, hd))
    return e;
  if (n_blocks == 0 || n_tokens == 0) return 0;
  if (!out || !lse || !dout || !delta || !dq || !dkp || !dvp) return DK_ERR_INVALID;
  if (!dk_aligned(out, 16) || !dk_aligned(dout, 16) || !dk_aligned(lse, 4) ||
      !dk_aligned(delta, 4) || !dk_aligned(dq, 16) || !dk_aligned(dkp, 4) || !dk_aligned(dvp, 4))
    return DK_ERR_ALIGN;
  const int64_t pairs = n_tokens * nq;
  hipLaunchKernelGGL(attn_delta_kernel, dim3((unsigned)((pairs + 15) / 16)), dim3(kAThreads), 0,
                     stream, (const f16*)out, (const f16*)dout, delta, n_tokens, nq);
  DK_CHECK_LAUNCH();
  hipLaunchKernelGGL(attn_dkdv_kernel, dim3((unsigned)n_blocks, (unsigned)nq), dim3(kAThreads), 0,
                     stream, a, (const f16*)dout, lse, delta, dkp, dvp);
  DK_CHECK_LAUNCH();
  hipLaunchKernelGGL(attn_dq_kernel, dim3((unsigned)n_blocks, (unsigned)nq), dim3(kAThreads), 0,
                     stream, a, (const f16*)dout, lse, delta, dq);
  DK_CHECK_LAUNCH();
  return 0;
}
