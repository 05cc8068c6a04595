// Attention forward on gfx950 (replaces solution/k_attn.py:40-83): causal GQA over the packed
// sequences with an online softmax in the exp2 domain.  Built with the MFMA accumulators in
// VGPRs (the build passes -amdgpu-mfma-vgpr-form for this file): in AGPRs the compiler copied
// the output accumulator out and back on every key tile.
#include "attn_dev.h"

namespace {

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
    // softmax of tile t in the exp2 domain.  Only tiles that reach the block's first query (the
    // diagonal, and the sequence end, which lies beyond it) hold masked keys: the test is uniform,
    // and key n = n0 + off + 4 (l / 32) is kept iff off <= min(m, seqlen - 1) - n0 - 4 (l / 32).
    if (n0 + kBN > mstart) {
      const int lim = (m < seqlen - 1 ? m : seqlen - 1) - n0 - 4 * hl;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          sc[kb][v] = kb * 32 + 8 * (v >> 2) + (v & 3) <= lim ? sc[kb][v] : -1.0e30f;
    }
    // the row maximum of the raw scores, scaled once (the scaling is monotonic)
    float mx = -1.0e30f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sc[kb][v]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // m_i is the reference point of l_i and O, not the exact running maximum: it moves (and O and
    // l are rescaled) only when some lane's maximum exceeds it by more than 2^8, so p =
    // 2^(s * qk_scale - m_i) stays below 256 (exact in fp16 to the same relative precision as
    // p <= 1) and the rescale, a read-modify-write of all of O, runs on the first tile and rarely
    // after.  The decision is per wave, so the branch is uniform.
    const float mt = __fmul_rn(mx, a.qk_scale);
    if (__builtin_amdgcn_ballot_w64(mt > m_i + 8.0f) != 0) {
      const float m_new = fmaxf(m_i, mt);
      const float alpha = ex2(__fsub_rn(m_i, m_new));
      l_i = __fmul_rn(l_i, alpha);
      m_i = m_new;
#pragma unroll
      for (int hb = 0; hb < kHD / 32; ++hb)
#pragma unroll
        for (int v = 0; v < 16; ++v) oacc[hb][v] = __fmul_rn(oacc[hb][v], alpha);
    }
    float rs = 0.0f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const float p = ex2(__builtin_fmaf(sc[kb][v], a.qk_scale, -m_i));
        sc[kb][v] = p;
        rs = __fadd_rn(rs, p);
      }
    rs = __fadd_rn(rs, __shfl_xor(rs, 32));
    l_i = __fadd_rn(l_i, rs);
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
  // result register v of block hb: head column hb * 32 + 8 (v / 4) + 4 (l / 32) + v % 4; one
  // correctly rounded reciprocal per row, then a product per element.  The wave's 32 x 128 block
  // of O is staged in its part of the K stages (free after the loop's last barrier) and written
  // back 16 bytes per lane, four whole 256-byte rows per store instruction: stored from the
  // registers, each instruction would cover 16 bytes of each of 32 rows' cache lines.
  constexpr int kOStride = kHD + 8;   // halves per staged row
  static_assert(kAThreads / 64 * 32 * kOStride <= kFwdStages * kTileHalves, "O staging in Ks");
  f16* ostage = Ks + w * 32 * kOStride;
  const float inv_l = __fdiv_rn(1.0f, l_i);   // rows past the sequence: not stored
#pragma unroll
  for (int hb = 0; hb < kHD / 32; ++hb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      f16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = (f16)__fmul_rn(oacc[hb][4 * g + e], inv_l);
      *reinterpret_cast<f16x4*>(ostage + c * kOStride + hb * 32 + 8 * g + 4 * hl) = o;
    }
  if (mval && hl == 0) lse[(int64_t)h * a.n_tokens + s0 + m] = __fadd_rn(m_i, log2f(l_i));
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4), cc = lane & 15;
    const int row = mstart + 32 * w + r;
    const f16x8 v = *reinterpret_cast<const f16x8*>(ostage + r * kOStride + 8 * cc);
    if (row < seqlen && s0 + row < a.n_tokens)
      *reinterpret_cast<f16x8*>(out + (s0 + row) * (int64_t)(a.nq * kHD) + h * kHD + 8 * cc) = v;
  }
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
