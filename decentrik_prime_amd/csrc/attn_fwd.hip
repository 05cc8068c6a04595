// Attention forward on gfx950 (replaces solution/k_attn.py:40-83): causal GQA over the packed
// sequences with an online softmax in the exp2 domain.  Built with the MFMA accumulators in
// VGPRs (the build passes -amdgpu-mfma-vgpr-form for this file): in AGPRs the compiler copied
// the output accumulator out and back on every key tile.
#include "attn_dev.h"

namespace {

// forward (solution/k_attn.py:40-83): one workgroup per (block of kBM queries, query head), 8
// waves: wave w takes queries 32 (w % 4) .. + 31 of the block and the key tiles t with
// t % 2 == w / 4, so two waves share each SIMD and each walks half of the block's tiles (the
// causal blocks walk 2 to 8 tiles of 64 keys).  The two halves' softmax states (running maximum,
// sum, O) are merged through LDS at the end.  Measured on MI355X at 4 x 512 tokens against 4
// waves each walking every tile (one wave per SIMD): 19.7 -> 18.5 us.
constexpr int kFThreads = 512;
constexpr int kFLoads = kTileHalves / 8 / kFThreads;   // DMA instructions per operand per lane: 2

__global__ __launch_bounds__(kFThreads) void attn_fwd_kernel(AttnArgs a, f16* __restrict__ out,
                                                             float* __restrict__ lse) {
  int64_t s0;
  int seqlen, mstart;
  if (!block_of(a, blockIdx.x, &s0, &seqlen, &mstart)) return;
  const int h = blockIdx.y;
  const int lane = threadIdx.x & 63, hl = lane >> 5, c = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int qw = wave & 3, kg = wave >> 2;   // query group, key-tile parity
  const int64_t ROW = (int64_t)(a.nq + 2 * a.nkv) * kHD;
  const int kvh = h / (a.nq / a.nkv);
  const int m = mstart + 32 * qw + c;
  const bool mval = m < seqlen && s0 + m < a.n_tokens;
  __shared__ __attribute__((aligned(1024))) f16 Ks[kFwdStages * kTileHalves];
  __shared__ __attribute__((aligned(1024))) f16 Vs[kFwdStages * kTileHalves];

  f32x16 oacc[kHD / 32];
#pragma unroll
  for (int hb = 0; hb < kHD / 32; ++hb) oacc[hb] = zero16();
  float m_i = -1.0e30f, l_i = 0.0f;
  const int hi = mstart + kBM < seqlen ? mstart + kBM : seqlen;
  const int n_tiles = (hi + kBN - 1) / kBN;
  const int n_pairs = (n_tiles + 1) / 2;
  const f16* kbase = a.qkv + s0 * ROW + (int64_t)(a.nq + kvh) * kHD;
  const f16* vbase = a.qkv + s0 * ROW + (int64_t)(a.nq + a.nkv + kvh) * kHD;
  // tile t into stage t % 4: instruction i of wave w fills the stage's chunks (8 i + w) 64 + lane,
  // row q / 16 (rows past the sequence read its last row: finite, and masked to p = 0)
  auto issue = [&](int t) {
    const int st = t % kFwdStages;
#pragma unroll
    for (int i = 0; i < kFLoads; ++i) {
      const int q = (8 * i + wave) * 64 + lane, r = q >> 4;
      const int row = t * kBN + r < seqlen ? t * kBN + r : seqlen - 1;
      const int64_t src = (int64_t)row * ROW + (((q & 15) ^ swz16(r)) << 3);
      const int dst = st * kTileHalves + (8 * i + wave) * 512;
      dma16(kbase + src, __builtin_amdgcn_readfirstlane(lds_addr(Ks + dst)));
      dma16(vbase + src, __builtin_amdgcn_readfirstlane(lds_addr(Vs + dst)));
    }
  };
  // tile pair u = tiles 2 u, 2 u + 1: pair 0 now, pair 1 after the query loads
  issue(0);
  if (n_tiles > 1) issue(1);
  // this lane's query row as the B operand (rows past the sequence: zeros).  Loaded at a clamped
  // row unconditionally and selected at once, so the compiler's wait for these loads stands here
  // (it then also covers pair 0, issued above) and not inside the loop.
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
  wait_vmem<0>();
  if (n_tiles > 2) issue(2);
  if (n_tiles > 3) issue(3);
  __syncthreads();
  for (int u = 0; u < n_pairs; ++u) {
    const int t = 2 * u + kg;
    if (t < n_tiles) {
      const f16* Kt = Ks + (t % kFwdStages) * kTileHalves;
      const f16* Vt = Vs + (t % kFwdStages) * kTileHalves;
      const int n0 = t * kBN;
      // S^T = K Q^T: keys kb * 32 + (row of the result), queries on the lanes
      f32x16 sc[2];
      sc[0] = sc[1] = zero16();
#pragma unroll
      for (int s = 0; s < kHD / 16; ++s)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          sc[kb] = mfma(*reinterpret_cast<const f16x8*>(Kt + sw_off(kb * 32 + c, 16 * s + 8 * hl)),
                        qf[s], sc[kb]);
      // keys past this lane's query (or the sequence end) masked: key n = n0 + off + 4 (l / 32)
      // is kept iff off <= min(m, seqlen - 1) - n0 - 4 (l / 32).  Only tiles that reach the
      // block's first query hold masked keys (the test is uniform).  A lane can see a tile whose
      // keys are all masked before any kept key (this wave skips every other tile): its masked
      // probabilities are set to 0 below rather than computed from the running maximum.
      const int lim = (m < seqlen - 1 ? m : seqlen - 1) - n0 - 4 * hl;
      const bool diag = n0 + kBN > mstart;
      if (diag) {
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
      // m_i is the reference point of l_i and O, not the exact running maximum: it moves (and O
      // and l are rescaled) only when some lane's maximum exceeds it by more than 2^8, so p =
      // 2^(s * qk_scale - m_i) stays below 256 and the rescale, a read-modify-write of all of O,
      // runs on the first tile and rarely after.  The decision is per wave (uniform branch).
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
          const bool kept = !diag || kb * 32 + 8 * (v >> 2) + (v & 3) <= lim;
          const float p = kept ? ex2(__builtin_fmaf(sc[kb][v], a.qk_scale, -m_i)) : 0.0f;
          sc[kb][v] = p;
          rs = __fadd_rn(rs, p);
        }
      rs = __fadd_rn(rs, __shfl_xor(rs, 32));
      l_i = __fadd_rn(l_i, rs);
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
    }
    // pair u + 1 landed (this wave's loads) and visible to every wave, and every wave is done
    // with pair u's stages, which then receive pair u + 2
    wait_vmem<0>();
    __syncthreads();
    if (2 * u + 4 < n_tiles) issue(2 * u + 4);
    if (2 * u + 5 < n_tiles) issue(2 * u + 5);
  }
  // merge: the odd-tile wave of each query group hands its state (O lane-major, 16 KB per wave,
  // in the K stages; m and l in the V stages' last KB) to the even-tile wave, which combines
  // O = O0 2^(m0 - m) + O1 2^(m1 - m), l likewise, m = max(m0, m1).  Every stage is free after
  // the loop's last barrier.
  float* ohand = reinterpret_cast<float*>(Ks) + qw * (kHD / 32) * 16 * 64;
  float* mlhand = reinterpret_cast<float*>(Vs) + (kFwdStages * kTileHalves / 2 - 256) + qw * 64;
  static_assert(4 * (kHD / 32) * 16 * 64 * 4 <= kFwdStages * kTileHalves * 2, "O hand-over in Ks");
  if (kg == 1) {
#pragma unroll
    for (int hb = 0; hb < kHD / 32; ++hb)
#pragma unroll
      for (int v = 0; v < 16; ++v) ohand[(hb * 16 + v) * 64 + lane] = oacc[hb][v];
    if (hl == 0) {
      mlhand[c] = m_i;
      mlhand[32 + c] = l_i;
    }
  }
  __syncthreads();
  // result register v of block hb: head column hb * 32 + 8 (v / 4) + 4 (l / 32) + v % 4; one
  // correctly rounded reciprocal per row, then a product per element.  The query group's 32 x 128
  // block of O is staged in the V stages (clear of the hand-over) and written back 16 bytes per
  // lane, four whole 256-byte rows per store instruction.
  constexpr int kOStride = kHD + 8;   // halves per staged row
  static_assert(4 * 32 * kOStride + 512 <= kFwdStages * kTileHalves, "O staging in Vs");
  f16* ostage = Vs + qw * 32 * kOStride;
  if (kg == 0) {
    const float m1 = mlhand[c], l1 = mlhand[32 + c];
    const float mm = fmaxf(m_i, m1);
    const float a0 = ex2(__fsub_rn(m_i, mm)), a1 = ex2(__fsub_rn(m1, mm));
    const float l = __fadd_rn(__fmul_rn(l_i, a0), __fmul_rn(l1, a1));
    const float inv_l = __fdiv_rn(1.0f, l);   // rows past the sequence: not stored
#pragma unroll
    for (int hb = 0; hb < kHD / 32; ++hb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int v = 4 * g + e;
          const float ov = __fadd_rn(__fmul_rn(oacc[hb][v], a0),
                                     __fmul_rn(ohand[(hb * 16 + v) * 64 + lane], a1));
          o[e] = (f16)__fmul_rn(ov, inv_l);
        }
        *reinterpret_cast<f16x4*>(ostage + c * kOStride + hb * 32 + 8 * g + 4 * hl) = o;
      }
    if (mval && hl == 0) lse[(int64_t)h * a.n_tokens + s0 + m] = __fadd_rn(mm, log2f(l));
  }
  __syncthreads();
  // the two waves of a query group store 16 of its 32 rows each
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * kg + 4 * i + (lane >> 4), cc = lane & 15;
    const int row = mstart + 32 * qw + r;
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
  hipLaunchKernelGGL(attn_fwd_kernel, dim3((unsigned)n_blocks, (unsigned)nq), dim3(kFThreads), 0,
                     stream, a, (f16*)out, lse);
  DK_CHECK_LAUNCH();
  return 0;
}
