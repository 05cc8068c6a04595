// Attention backward on gfx950 (replaces solution/k_attn.py:84-245): delta, dK/dV per query
// head, dQ; the shared layout and helpers are in attn_dev.h.
#include "attn_dev.h"

namespace {

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
__device__ __forceinline__ void dq_block(const AttnArgs& a, int blk, int h,
                                         const f16* __restrict__ dout,
                                         const float* __restrict__ lse,
                                         const float* __restrict__ delta, float* __restrict__ dq,
                                         f16* Ks, f16* Vs) {
  int64_t s0;
  int seqlen, mstart;
  if (!block_of(a, blk, &s0, &seqlen, &mstart)) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, hl = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(w);
  const int64_t ROW = (int64_t)(a.nq + 2 * a.nkv) * kHD, OROW = (int64_t)a.nq * kHD;
  const int kvh = h / (a.nq / a.nkv);
  const int m = mstart + 32 * w + c;
  const bool mval = m < seqlen && s0 + m < a.n_tokens;

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
    // P and dS^T = P (dP^T - delta).  Rows past the sequence have zero q, dO and delta, so their
    // dS is zero whatever P is; keys past a query or the sequence are masked only on the tiles
    // that reach this wave's first query (a wave-uniform test): key n = n0 + off + 4 (l / 32) is
    // kept iff off <= min(m, seqlen - 1) - n0 - 4 (l / 32).  The exponential is computed for
    // every score and then selected (a conditional exponential becomes a branch).
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        sc[kb][v] = ex2(__builtin_fmaf(sc[kb][v], a.qk_scale, -lse_m));
    if (n0 + kBN - 1 > mstart + 32 * wave || n0 + kBN > seqlen) {
      const int lim = (m < seqlen - 1 ? m : seqlen - 1) - n0 - 4 * hl;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          sc[kb][v] = kb * 32 + 8 * (v >> 2) + (v & 3) <= lim ? sc[kb][v] : 0.0f;
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) sc[kb][v] = __fmul_rn(sc[kb][v], __fsub_rn(dc[kb][v], dl_m));
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
  // the wave's 32 x 128 block of dQ staged in the (now free) tile ring, waves 0-1 in the K stages
  // and 2-3 in the V stages, then written back 16 bytes per lane, two whole 512-byte rows per
  // store instruction (stored from the registers, each instruction would cover 32 bytes of each
  // of 32 rows' cache lines); rows past the sequence are not stored
  constexpr int kQStride = kHD + 4;   // floats per staged row
  static_assert(2 * 32 * kQStride * 4 <= kFwdStages * kTileHalves * 2, "dQ staging in the ring");
  float* qstage = reinterpret_cast<float*>(w < 2 ? Ks : Vs) + (w & 1) * 32 * kQStride;
#pragma unroll
  for (int hb = 0; hb < kHD / 32; ++hb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = __fmul_rn(dqacc[hb][4 * g + e], a.sm_scale);
      *reinterpret_cast<f32x4*>(qstage + c * kQStride + hb * 32 + 8 * g + 4 * hl) = o;
    }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int r = 2 * i + hl, row = mstart + 32 * w + r;
    const f32x4 v = *reinterpret_cast<const f32x4*>(qstage + r * kQStride + 4 * c);
    if (row < seqlen && s0 + row < a.n_tokens)
      *reinterpret_cast<f32x4*>(dq + (s0 + row) * OROW + h * kHD + 4 * c) = v;
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

__device__ __forceinline__ void dkdv_block(const AttnArgs& a, int blk, int h,
                                           const f16* __restrict__ dout,
                                           const float* __restrict__ lse,
                                           const float* __restrict__ delta,
                                           float* __restrict__ dkp, float* __restrict__ dvp,
                                           f16* Qs, f16* Ds, float (*lse_s)[kBN],
                                           float (*dl_s)[kBN]) {
  int64_t s0;
  int seqlen, nstart;
  if (!block_of(a, blk, &s0, &seqlen, &nstart)) return;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, hl = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(w);
  const int64_t ROW = (int64_t)(a.nq + 2 * a.nkv) * kHD, OROW = (int64_t)a.nq * kHD;
  const int kvh = h / (a.nq / a.nkv);
  const int n = nstart + 32 * w + c;   // this lane's key
  const bool nval = n < seqlen && s0 + n < a.n_tokens;

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
    // the statistics of this lane's 32 queries of the tile: rows qb * 32 + 8 g + 4 (l / 32) + 0..3
    f32x4 ls[2][4], ds[2][4];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        ls[qb][g] = *reinterpret_cast<const f32x4*>(&lse_s[st][qb * 32 + 8 * g + 4 * hl]);
        ds[qb][g] = *reinterpret_cast<const f32x4*>(&dl_s[st][qb * 32 + 8 * g + 4 * hl]);
      }
    // P, computed for every score and then selected (a conditional exponential becomes a branch).
    // Keys past the sequence only reach rows of dK and dV that are not stored; queries before a
    // key or past the sequence are masked only on the tiles that hold such a query for this wave
    // (a wave-uniform test): query q = m0 + off + 4 (l / 32) is kept iff lo <= off < hi.
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int v = 0; v < 16; ++v)
        sc[qb][v] = ex2(__builtin_fmaf(sc[qb][v], a.qk_scale, -ls[qb][v >> 2][v & 3]));
    if (m0 < nstart + 32 * wave + 31 || m0 + kBN > seqlen) {
      const int lo = n - m0 - 4 * hl, hi = seqlen - m0 - 4 * hl;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int off = qb * 32 + 8 * (v >> 2) + (v & 3);
          sc[qb][v] = ((off >= lo) & (off < hi)) ? sc[qb][v] : 0.0f;
        }
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int v = 0; v < 16; ++v)   // dS
        dc[qb][v] = __fmul_rn(sc[qb][v], __fsub_rn(dc[qb][v], ds[qb][v >> 2][v & 3]));
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

// dK/dV and dQ in one launch.  Workgroups [0, n_blocks * nq) run the dK/dV blocks in block-table
// order, the rest the dQ blocks in reverse block-table order, each with every head of a block
// before the next block.  The hardware deals workgroups to the 8 XCDs round-robin and each XCD
// starts its own in index order, so with a table whose blocks are ordered by the rows from their
// start to their sequence's end, longest first (the dK/dV walk; reversed, the dQ walk for sequences
// of equal length), every XCD gets a balanced share, started longest first: the dQ blocks begin
// on the CUs the dK/dV blocks leave idle and then on those that short blocks free.  Any table
// order gives the same results.  Both read delta, which the launch before computes.
__global__ __launch_bounds__(kAThreads) void attn_bwd_kernel(AttnArgs a, const f16* __restrict__ dout,
                                                             const float* __restrict__ lse,
                                                             const float* __restrict__ delta,
                                                             float* __restrict__ dq,
                                                             float* __restrict__ dkp,
                                                             float* __restrict__ dvp, int n_blocks) {
  static_assert(kBwdStages == kFwdStages, "dK/dV and dQ share the tile ring");
  __shared__ __attribute__((aligned(1024))) f16 T0[kBwdStages * kTileHalves];
  __shared__ __attribute__((aligned(1024))) f16 T1[kBwdStages * kTileHalves];
  __shared__ __attribute__((aligned(16))) float lse_s[kBwdStages][kBN], dl_s[kBwdStages][kBN];
  const int per = n_blocks * a.nq;
  const int g = blockIdx.x;
  if (g < per)
    dkdv_block(a, g / a.nq, g % a.nq, dout, lse, delta, dkp, dvp, T0, T1, lse_s, dl_s);
  else
    dq_block(a, n_blocks - 1 - (g - per) / a.nq, (g - per) % a.nq, dout, lse, delta, dq, T0, T1);
}

}  // namespace

extern "C" int dk_attn_bwd(const void* qkv, const void* out, const float* lse, const void* dout,
                           const int32_t* cu_seqlens, int32_t n_seq, const int32_t* block_table,
                           int32_t n_blocks, int64_t n_tokens, int32_t nq, int32_t nkv, int32_t hd,
                           float* delta, float* dq, float* dkp, float* dvp, hipStream_t stream) {
  AttnArgs a;
  if (int e = attn_args(a, qkv, cu_seqlens, n_seq, block_table, n_blocks, n_tokens, nq, nkv, hd))
    return e;
  if (n_blocks == 0 || n_tokens == 0) return 0;
  if (!out || !lse || !dout || !delta || !dq || !dkp || !dvp) return DK_ERR_INVALID;
  if (2 * (int64_t)n_blocks * nq > INT32_MAX) return DK_ERR_INVALID;   // one workgroup index
  if (!dk_aligned(out, 16) || !dk_aligned(dout, 16) || !dk_aligned(lse, 4) ||
      !dk_aligned(delta, 4) || !dk_aligned(dq, 16) || !dk_aligned(dkp, 4) || !dk_aligned(dvp, 4))
    return DK_ERR_ALIGN;
  const int64_t pairs = n_tokens * nq;
  hipLaunchKernelGGL(attn_delta_kernel, dim3((unsigned)((pairs + 15) / 16)), dim3(kAThreads), 0,
                     stream, (const f16*)out, (const f16*)dout, delta, n_tokens, nq);
  DK_CHECK_LAUNCH();
  hipLaunchKernelGGL(attn_bwd_kernel, dim3((unsigned)(2 * n_blocks * nq)), dim3(kAThreads), 0,
                     stream, a, (const f16*)dout, lse, delta, dq, dkp, dvp, n_blocks);
  DK_CHECK_LAUNCH();
  return 0;
}
