// fp16-weight GEMMs with the fused epilogues on 256 x 256 tiles (gfx950).
//
//   NT (TRANS = false): C[m][n] = sum_k A[m][k] * W[n][k]      W = p.w16 stored [N][K]
//   NN (TRANS = true):  C[m][n] = sum_k A[m][k] * W[k][n]      W = p.w16 stored [K][N]
//
// One 512-thread workgroup per CU owns a 256 x 256 tile of C: 8 waves (2 x 4), each a 128 x 64
// block of v_mfma_f32_16x16x32_f16 results.  Per output FLOP that is half the operand bytes of a
// 128 x 128 tile.  With real operand data these GEMMs run at the clock that the power limit
// allows, so energy per FLOP sets their rate: the 16 x 16 x 32 MFMA takes less of it than the
// 32 x 32 x 16 one.  K is walked in steps of 64.  Operands go from global memory straight into
// LDS with global_load_lds_dwordx4 (LDS DMA: no registers, no LDS write instructions) into two
// stages (2 x 64 KB): the loads of step k + 2 go out during the last MFMAs of step k, into the
// stage step k has just finished reading.  Each wave waits only for its own loads (vmcnt), and
// one barrier per step both publishes the next step's tiles and frees the stage just read.  The
// MFMA operands of the next 32-wide sub-step are read while the MFMAs of the current one run; the
// last sub-step, which issues the refill, runs at wave priority 1 so that its loads go out ahead
// of the other wave's operand reads.  (Measured on MI355X: 64-wide steps in two stages run about
// 8% faster than 32-wide steps in a four-stage ring; the barriers, not the load distance, are
// what costs.)  With W4 = true the workgroup builds each step's W tile itself from the packed NF4
// weight (dequantised in registers beside the MFMAs and written into the stage), bit-identical
// to the fp16-weight form.
//
// LDS layout: A tiles and NT W tiles are rows of 64 halves (128 bytes) whose eight 16-byte
// chunks are XOR-swizzled by row (swz_k), so the b128 operand reads hit no bank conflict.  NN W
// tiles are rows of 256 halves (N contiguous) with chunks swizzled by k (swz_n); the
// consumers build each K-contiguous operand from two ds_read_b64_tr_b16 (transposing) reads.
// The DMA writes 64 consecutive 16-byte chunks per instruction, so the swizzle is applied to the
// global addresses each lane loads.
//
// Tiles are dealt M-fastest inside each XCD's contiguous run of workgroups.  When the tile count
// leaves a last round at most half full, those last tiles run as four 128 x 128 sub-tiles each
// (8 waves of 32 x 64), so the final round is short instead of mostly idle; in the SwiGLU
// backward they are dispatched first, which staggers the rounds' HBM-bound epilogues.  The fp16
// SwiGLU GEMMs, whose tiles take more than one round, run one persistent workgroup per CU that
// walks the same tiles in the same order, overlapping each tile's first loads with the previous
// tile's epilogue stores.
//
// Epilogues as in w4gemm.hip (the same per-element rounding): LINEAR with up to two LoRA terms
// and the three output modes, SWIGLU_FWD (gate/up rows interleaved in groups of 32 so g and u of
// an output share a lane), SWIGLU_BWD (in place on gu).
//
// A launch may carry NF4 dequant work (GemmParams::side, nf4_dev.h) on extra workgroups after the
// tiles: the hardware dispatches workgroups in order, so they start on the CUs that a last round
// of tiles (or a grid smaller than the CU count) leaves idle, and the dequant of the next layer's
// weights runs under this GEMM instead of in a launch of its own.
#include "gemm_common.h"

namespace dk {
namespace {

typedef float f32x8_t __attribute__((ext_vector_type(8)));

constexpr int kBK = 64;                      // K per step
constexpr int kStages = 2;                   // LDS stages
constexpr int kThreads = 512;
constexpr int kTile = 256;
constexpr int kStageHalves = kTile * kBK;    // one operand of one stage: 32 KB
constexpr int kEpiScratch = 16384;           // bytes of LDS per wave for the epilogue

// Epilogue scratch of a wave with TN 32-column blocks per strip: the staged strip (32 rows of
// 32 TN + 4 floats) plus the keep-mask and LoRA A slices (1536 bytes each).
constexpr int epi_scratch_bytes(int tn) { return 32 * (32 * tn + 4) * 4 + 3072; }

__device__ __forceinline__ unsigned lds_offset(const void* p) {
  return (unsigned)(size_t)(__attribute__((address_space(3))) const void*)p;
}

// 16 bytes per lane from global memory into LDS at lds + 16 * lane.  Written as inline assembly
// so that the compiler does not guard every later LDS read with a wait for it: the kernel tracks
// these loads itself with vmcnt waits.  M0 (the LDS address) is saved and restored around it.
// The SADDR form: the global address is a wave-uniform 64-bit base held in SGPRs plus a 32-bit
// unsigned byte offset per lane.  One address register per lane instead of two and no per-load
// address arithmetic (the base advances by whole K steps in scalar registers): in a
// microbenchmark of the main loop on MI355X the loads cost 12.5 % of the MFMA issue cycles in
// this form against 20 % with a 64-bit address per lane.
__device__ __forceinline__ void dma16s(uint64_t base, unsigned off, unsigned lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, %3\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(off), "s"(base)
      : "memory");
}

// A wave-uniform 64-bit value in scalar registers.  readfirstlane returns int: each half goes
// through uint32_t so that the low half is zero-extended.
__device__ __forceinline__ uint64_t uniform64(uint64_t v) {
  return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((unsigned)(v >> 32)) << 32) |
         (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((unsigned)v);
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

__device__ __forceinline__ f16x4 read_tr(const f16* p) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                       (__attribute__((address_space(3))) i16x4*)(p)));
}

// Chunk swizzles, the 16-byte chunk index of a row XORed with a function of the row: rows of
// 64 halves (A tiles, NT W tiles; swz_k) and N-contiguous rows of the NN W tile (swz_n).  Chosen by
// measurement (the SQ_LDS_BANK_CONFLICT counter on MI355X, each candidate in a loop of the
// GEMM's operand reads): conflict-free for both operand patterns, the 16x16x32 one (lane l: row
// l % 16, chunk 4 s + l / 16; NN: 16-lane groups reading rows 8 g + 4 h + 0..3) and the 32x32x16
// one (row l % 32, chunk 2 q + l / 32; NN: rows 8 (l / 32) + 4 h + 0..3).  The earlier
// (r & 7) ^ (r >> 3 & 1) and 4 (k & 3) were conflict-free for the second only (two-way conflicts
// for the first).
__device__ __forceinline__ int swz_k(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 2); }
__device__ __forceinline__ int swz_n(int k) { return (4 * (k & 3)) ^ (2 * ((k >> 3) & 1)); }

// The fused epilogue of one wave's TM x TN blocks of 32 x 32 results, whose top-left output
// element is (mw0, nw0).  A block is four 16 x 16 v_mfma_f32_16x16x32_f16 results: register v of
// lane l holds row 16 (v / 8) + 4 (l / 16) + v % 4, column 16 (v / 4 % 2) + l % 16.  Each 32-row
// strip i is finished in registers (bias, LoRA terms, fp16 rounding), staged in this wave's LDS
// scratch `escr` (epi_scratch_bytes(TN) bytes) and written back as 16-byte vectors of 8
// consecutive columns, so that the global traffic (and the gate/up reads of the SwiGLU backward)
// moves in whole 16-byte pieces.
template <bool TRANS, int EPI, int TM, int TN>
__device__ __forceinline__ void wave_epilogue(const GemmParams& p, f32x16 (&acc)[TM][TN],
                                              int64_t mw0, int64_t nw0, uint8_t* escr,
                                              const uint8_t* pscr) {
  constexpr int COLS = 32 * TN;          // columns of a strip
  // floats per staged row: the four row groups a staging store covers (rows 4 apart) land 16
  // banks apart, so the stores are free of bank conflicts (measured with SQ_LDS_BANK_CONFLICT on
  // MI355X: rows of COLS + 8 floats with the 16-byte chunks of odd rows swapped in pairs, the
  // previous layout, cost these stores two-way conflicts; the read-backs cost the same either way)
  constexpr int SLD = COLS + 4;
  constexpr int SEGS = COLS / 8;         // 8-column segments per row
  constexpr int ROWS_PER_PASS = 64 / SEGS;
  static_assert(32 * SLD * 4 + 3072 == epi_scratch_bytes(TN) && epi_scratch_bytes(TN) <= kEpiScratch,
                "epilogue scratch");
  const int lane = threadIdx.x & 63;
  const int lc = lane & 15;          // column in a 16-column block
  const int lk4 = 4 * (lane >> 4);   // first row in a 16-row block; first rank of a LoRA MFMA
  auto erow = [&](int v) { return 16 * (v >> 3) + lk4 + (v & 3); };
  auto ecol = [&](int v) { return 16 * ((v >> 2) & 1) + lc; };
  const int64_t M = p.M, N = p.N;
  float* stage = reinterpret_cast<float*>(escr);
  uint8_t* mscr = escr + 32 * SLD * 4;   // keep-mask bytes (rows of 48 bytes)
  f16* ascr = reinterpret_cast<f16*>(mscr + 1536);   // LoRA A slice (rows of 48 halves)
  const int seg = lane % SEGS, srow = lane / SEGS;   // read-back position of this lane

  // registers -> staged strip (the values, already rounded where the output is fp16)
  auto stage_block = [&](int j, const f32x16& r) {
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      stage[erow(v) * SLD + 32 * j + ecol(v)] = r[v];
    }
  };
  auto staged8_of = [&](const float* st, int row, int col) {
    const f32x4 a = *reinterpret_cast<const f32x4*>(st + row * SLD + col);
    const f32x4 b = *reinterpret_cast<const f32x4*>(st + row * SLD + col + 4);
    return f32x8_t{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  };
  auto staged8 = [&](int row, int col) { return staged8_of(stage, row, col); };

  // SwiGLU backward: the gate/up rows of strip i + 1 are loaded while strip i is finished (two
  // buffers), so that one strip's HBM round trip stands on the tile's path instead of TM
  constexpr int BPASSES = 32 / ROWS_PER_PASS;
  constexpr int BBUF = EPI == EPI_SWIGLU_BWD ? 2 : 1;
  f16x8 gqb[BBUF][BPASSES], uqb[BBUF][BPASSES];
  auto load_gu = [&](int i, int b) {
#pragma unroll
    for (int q = 0; q < BPASSES; ++q) {
      const int64_t m = mw0 + 32 * i + srow + q * ROWS_PER_PASS;
      const f16* gp = p.gu + (m < M ? m : M - 1) * 2 * p.inter + nw0 + 8 * seg;   // rows past M: unused
      gqb[b][q] = *reinterpret_cast<const f16x8*>(gp);
      uqb[b][q] = *reinterpret_cast<const f16x8*>(gp + p.inter);
    }
  };
  if constexpr (EPI == EPI_SWIGLU_BWD) load_gu(0, 0);

#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t mrow0 = mw0 + 32 * i;
    if constexpr (EPI == EPI_LINEAR) {
      f32x16 res[TN];
      float bias[TN][2];
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int h = 0; h < 2; ++h) bias[j][h] = p.bias ? (float)p.bias[nw0 + 32 * j + ecol(4 * h)] : 0.0f;
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          res[j][v] = (float)dk_h(__fadd_rn(acc[i][j][v], bias[j][(v >> 2) & 1]));
      // LoRA terms (at most two), in batches of TB: both at once for a single strip per wave
      // (128 x 128 tiles, registers to spare), one at a time otherwise.  Every global load a batch
      // needs in this strip (the z rows, the B rows or A columns of each block, the keep-mask
      // bytes) is issued, at rows clamped to M (rows past M are never stored), before the first
      // is used: one memory round trip per batch and 16 ranks.  Each 16 x 16 quarter of a block
      // takes one v_mfma_f32_16x16x16_f16 per 16 ranks (the result layout above).  The terms are
      // added to the result in order, as separate roundings.
      constexpr int TB = TM == 1 ? 2 : 1;
      int64_t zm[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int64_t r = mrow0 + 16 * h + lc;
        zm[h] = r < M ? r : M - 1;
      }
      for (int t0 = 0; t0 < p.n_lora; t0 += TB) {
        bool on[TB][TN], masked[TB];
        f32x4 lo[TB][TN][4];   // quarter 2 (row half) + (column half)
        u32x4 mw[TB][TN];
#pragma unroll
        for (int b = 0; b < TB; ++b) {
          const LoraTerm& L = p.lora[t0 + b < 2 ? t0 + b : 1];
          const bool live = t0 + b < p.n_lora;
          masked[b] = TRANS && live && L.mask;
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            on[b][j] = live && (TRANS || (nw0 + 32 * j >= L.n_begin && nw0 + 32 * j < L.n_end));
#pragma unroll
            for (int q = 0; q < 4; ++q) lo[b][j][q] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          }
          if (masked[b]) {
            // the blocks' 32 x 32 keep-mask bytes: one 16-byte load per lane and block
            const int64_t mr = mrow0 + (lane >> 1) < M ? mrow0 + (lane >> 1) : M - 1;
#pragma unroll
            for (int j = 0; j < TN; ++j)
              mw[b][j] = *reinterpret_cast<const u32x4*>(L.mask + mr * N + nw0 + 32 * j +
                                                          16 * (lane & 1));
          }
        }
        for (int rc = 0; rc < p.rank; rc += 16) {
          // z rows (16 h + l % 16) and, NT, B rows of the lane's columns (32 j + 16 h + l % 16),
          // ranks rc + 4 (l / 16) ..; NN, A[rc + l / 4][8 columns of the block]
          f16x4 zf[TB][2], rr4[TB][TN][2];
          f16x8 rr8[TB][TN];
#pragma unroll
          for (int b = 0; b < TB; ++b) {
            if (t0 + b >= p.n_lora) continue;
            const LoraTerm& L = p.lora[t0 + b];
#pragma unroll
            for (int h = 0; h < 2; ++h)
              zf[b][h] = *reinterpret_cast<const f16x4*>(L.z + zm[h] * p.rank + rc + lk4);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
              if (!on[b][j]) continue;
              if (!TRANS) {
#pragma unroll
                for (int h = 0; h < 2; ++h)
                  rr4[b][j][h] = *reinterpret_cast<const f16x4*>(
                      L.r + (nw0 + 32 * j + 16 * h + lc - L.n_begin) * p.rank + rc + lk4);
              } else {
                rr8[b][j] = *reinterpret_cast<const f16x8*>(L.r + (int64_t)(rc + (lane >> 2)) * N +
                                                           nw0 + 32 * j + 8 * (lane & 3));
              }
            }
          }
#pragma unroll
          for (int b = 0; b < TB; ++b)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
              if (!on[b][j]) continue;
              f16x4 rf[2];
              if (TRANS) {
                // A[rc .. rc + 16][block columns] staged row-major (rows of 48 halves), read back
                // rank-contiguous with transposing reads: lane l gets column 16 h + l % 16, ranks
                // 4 (l / 16) .. + 3
                __builtin_amdgcn_wave_barrier();
                *reinterpret_cast<f16x8*>(ascr + (lane >> 2) * 48 + 8 * (lane & 3)) = rr8[b][j];
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int h = 0; h < 2; ++h)
                  rf[h] = __builtin_bit_cast(
                      f16x4, read_tr(ascr + (lk4 + (lc >> 2)) * 48 + 16 * h + 4 * (lane & 3)));
                __builtin_amdgcn_wave_barrier();
              } else {
                rf[0] = rr4[b][j][0];
                rf[1] = rr4[b][j][1];
              }
#pragma unroll
              for (int q = 0; q < 4; ++q)
                lo[b][j][q] = __builtin_amdgcn_mfma_f32_16x16x16f16(zf[b][q >> 1], rf[q & 1],
                                                                    lo[b][j][q], 0, 0, 0);
            }
        }
#pragma unroll
        for (int b = 0; b < TB; ++b)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            if (!on[b][j]) continue;
            const float sc = p.lora[t0 + b].scale;
            if (masked[b]) {
              // staged in LDS (rows of 48 bytes), then read per element
              __builtin_amdgcn_wave_barrier();
              *reinterpret_cast<u32x4*>(mscr + (lane >> 1) * 48 + 16 * (lane & 1)) = mw[b][j];
              __builtin_amdgcn_wave_barrier();
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const float lf = (float)dk_h(lo[b][j][v >> 2][v & 3]);
                res[j][v] = __fadd_rn(res[j][v], mscr[erow(v) * 48 + ecol(v)] ? __fmul_rn(lf, sc) : 0.0f);
              }
              __builtin_amdgcn_wave_barrier();
            } else {
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const float lf = (float)dk_h(lo[b][j][v >> 2][v & 3]);
                res[j][v] = __fadd_rn(res[j][v], TRANS ? lf : __fmul_rn(sc, lf));
              }
            }
          }
      }
      // rotary embedding (solution/k_rope.py:23-61): this wave's 64 columns are one half of a
      // head, the partner wave (whose scratch is pscr) holds the other half of the same rows;
      // the pair is rotated in fp32 from the staged values, then rounded once
      const bool rope = !TRANS && p.rope_pos != nullptr && nw0 < p.rope_cols;
      if (p.out_mode == DK_OUT_F16 && !rope) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v) res[j][v] = (float)dk_h(res[j][v]);
      }
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < TN; ++j) stage_block(j, res[j]);
      __builtin_amdgcn_wave_barrier();
      if (!TRANS && p.rope_pos) __syncthreads();   // every wave's strip is staged
#pragma unroll
      for (int q = 0; q < 32 / ROWS_PER_PASS; ++q) {
        const int row = srow + q * ROWS_PER_PASS;
        const int64_t m = mrow0 + row;
        if (m >= M) continue;
        f32x8_t r = staged8(row, 8 * seg);
        const int64_t o = m * p.ldo + nw0 + 8 * seg;
        if (rope) {
          const f32x8_t pr = staged8_of(reinterpret_cast<const float*>(pscr), row, 8 * seg);
          const float* ct = p.rope_cos + (int64_t)p.rope_pos[m] * p.rope_hd + 8 * seg;
          const float* sn = p.rope_sin + (int64_t)p.rope_pos[m] * p.rope_hd + 8 * seg;
          const f32x4 c0 = *reinterpret_cast<const f32x4*>(ct), c1 = *reinterpret_cast<const f32x4*>(ct + 4);
          const f32x4 s0 = *reinterpret_cast<const f32x4*>(sn), s1 = *reinterpret_cast<const f32x4*>(sn + 4);
          const float c8[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
          const float s8[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
          // first half: x1 c - x2 s (own x1); second half: x2 c + x1 s (own x2)
          const bool first = (nw0 % p.rope_hd) == 0;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float a = __fmul_rn(r[e], c8[e]), b = __fmul_rn(pr[e], s8[e]);
            r[e] = first ? __fsub_rn(a, b) : __fadd_rn(a, b);
          }
        }
        if (p.out_mode == DK_OUT_F16) {
          f16x8 h;
#pragma unroll
          for (int e = 0; e < 8; ++e) h[e] = rope ? dk_h(r[e]) : (f16)r[e];
          *reinterpret_cast<f16x8*>(reinterpret_cast<f16*>(p.out) + o) = h;
        } else {
          float* dst = reinterpret_cast<float*>(p.out) + o;
          f32x4 lo4 = f32x4{r[0], r[1], r[2], r[3]}, hi4 = f32x4{r[4], r[5], r[6], r[7]};
          if (p.out_mode == DK_OUT_F32_ACCUM) {
            const f32x4 p0 = *reinterpret_cast<const f32x4*>(dst);
            const f32x4 p1 = *reinterpret_cast<const f32x4*>(dst + 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              lo4[e] = __fadd_rn(p0[e], lo4[e]);
              hi4[e] = __fadd_rn(p1[e], hi4[e]);
            }
          }
          *reinterpret_cast<f32x4*>(dst) = lo4;
          *reinterpret_cast<f32x4*>(dst + 4) = hi4;
        }
      }
      __builtin_amdgcn_wave_barrier();
      if (!TRANS && p.rope_pos) __syncthreads();   // the partner has read this wave's strip
    } else if constexpr (EPI == EPI_SWIGLU_FWD) {
      // block 0: the gate values, block 1: the up values of the same 32 hidden units
      f32x16 g, u;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        g[v] = (float)dk_h(acc[i][0][v]);
        u[v] = (float)dk_h(acc[i][1][v]);
      }
      __builtin_amdgcn_wave_barrier();
      stage_block(0, g);
      stage_block(1, u);
      __builtin_amdgcn_wave_barrier();
      // 32 rows x 4 segments of 8 hidden units: 2 per lane
      const int hseg = lane & 3, hrow = lane >> 2;
      const int64_t hcol = nw0 / 2 + 8 * hseg;
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int row = hrow + 16 * q;
        const int64_t m = mrow0 + row;
        if (m >= M) continue;
        const f32x8_t gv = staged8(row, 8 * hseg), uv = staged8(row, 32 + 8 * hseg);
        f16x8 ah, gh, uh;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float sig, silu;
          dk_silu_parts(gv[e], &sig, &silu);
          ah[e] = dk_h(silu * uv[e]);
          gh[e] = (f16)gv[e];
          uh[e] = (f16)uv[e];
        }
        *reinterpret_cast<f16x8*>(reinterpret_cast<f16*>(p.out) + m * p.ldo + hcol) = ah;
        if (p.gu) {
          *reinterpret_cast<f16x8*>(p.gu + m * 2 * p.inter + hcol) = gh;
          *reinterpret_cast<f16x8*>(p.gu + m * 2 * p.inter + p.inter + hcol) = uh;
        }
      }
      __builtin_amdgcn_wave_barrier();
    } else {  // EPI_SWIGLU_BWD: N == inter; dact = fp16(acc), then the gated-SiLU backward on gu
      // (strips are disjoint row ranges, so the next strip's loads never read what this one
      // stores)
      if (i + 1 < TM) load_gu(i + 1, (i + 1) & 1);
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        f32x16 d;
#pragma unroll
        for (int v = 0; v < 16; ++v) d[v] = (float)dk_h(acc[i][j][v]);
        stage_block(j, d);
      }
      __builtin_amdgcn_wave_barrier();
      constexpr int PASSES = BPASSES;
      const f16x8(&gq)[PASSES] = gqb[i & (BBUF - 1)];
      const f16x8(&uq)[PASSES] = uqb[i & (BBUF - 1)];
#pragma unroll
      for (int q = 0; q < PASSES; ++q) {
        const int row = srow + q * ROWS_PER_PASS;
        const int64_t m = mrow0 + row;
        if (m >= M) continue;
        const f32x8_t da = staged8(row, 8 * seg);
        f16x8 dg, du;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float g = (float)gq[q][e], u = (float)uq[q][e];
          float sig, silu;
          dk_silu_parts(g, &sig, &silu);
          du[e] = dk_h(da[e] * silu);
          dg[e] = dk_h((da[e] * u) * sig * (1.0f + g * (1.0f - sig)));
        }
        f16* gp = p.gu + m * 2 * p.inter + nw0 + 8 * seg;
        *reinterpret_cast<f16x8*>(gp) = dg;
        *reinterpret_cast<f16x8*>(gp + p.inter) = du;
      }
      __builtin_amdgcn_wave_barrier();
    }
  }
}

// NST: LDS stages of this tile shape in the kernel's 2 x 64 KB (256 x 256: 2, 128 x 128: 4, so
// the smaller tiles, whose steps are a quarter as long, still load three steps ahead).
// 128 x 128 NT tiles of the fp16 weight split the waves by role in the main loop: waves 0-3
// compute (WAVES_M x 4 / WAVES_M blocks of 64 x 64: 16 MFMAs per 32-wide sub-step on eight
// operand reads) and never load or wait for loads; waves 4-7 issue every load of the tile and
// wait for them.  Each computing wave then hands its second 32-row strip to a loading wave, so
// the eight waves run the epilogue on one 32 x 64 strip each, as in the 8-wave tile.  Measured on
// MI355X: the loop alone (microbenchmark) 723 against 927 core clocks per 64-wide step (the MFMA
// work is 512); in the step q|k|v forward 24.4 -> 23.4 us, o forward 20.6 -> 18.8 us.  NN tiles
// keep the 8-wave form: specialised they ran faster alone but slower in the step (o dX
// 21.7 -> 22.6 us).  Every output element is summed by the same MFMA sequence either way.
template <bool TRANS, int EPI, int BM, int BN, int WAVES_M, int NST, bool W4>
__device__ __forceinline__ void gemm_tile(const GemmParams& p, int64_t m0, int64_t n0, int kt0,
                                          int nk, float* part, f16* As, f16* Bs,
                                          const float* w4tab) {
  constexpr int SA = BM * kBK, SB = BN * kBK;   // halves per stage of A and of W
  static_assert(NST * SA <= kStages * kStageHalves && NST * SB <= kStages * kStageHalves &&
                (NST & (NST - 1)) == 0 && NST >= 2, "LDS stages");
  constexpr bool SPEC = BM == 128 && BN == 128 && !W4 && !TRANS;   // waves split by role

  constexpr int NCW = SPEC ? 4 : 8;         // computing waves
  constexpr int NLW = SPEC ? 4 : 8;         // loading waves
  constexpr int WAVES_N = NCW / WAVES_M;
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int LA = BM * 8 / (64 * NLW);   // A chunks per loading lane per stage
  constexpr int LB = BN * 8 / (64 * NLW);   // W chunks per loading lane per stage
  constexpr int LOADS = W4 ? LA : LA + LB;  // DMA instructions per lane per stage (W4: A only)
  constexpr int NCH = BN / 8;               // NN: 16-byte chunks per W-tile row
  static_assert(TM >= 1 && TN >= 1 && LA >= 1 && LB >= 1, "tile shape");
  static_assert(EPI != EPI_SWIGLU_FWD || (TN == 2 && !TRANS), "SwiGLU forward needs WN = 64");

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t M = p.M, N = p.N, K = p.K;
  const bool loader = !SPEC || wave >= NCW;            // issues loads and waits for them
  const int lw = SPEC ? wave - NCW : wave;              // its index among the loading waves

  // ---- DMA sources (first K step kt0; nk steps): instruction j of loading wave w fills the
  // stage's chunks [(NLW j + w) 64, +64).  Each operand has a wave-uniform base at step kt0 (A:
  // the tile's first row; W: the weight's first row (NT) or the tile's first column (NN)) and a
  // 32-bit byte offset per lane and instruction; the host keeps every offset below 2^32.
  const uint64_t a_base = uniform64((uint64_t)(p.a + m0 * p.lda + (int64_t)kt0 * kBK));
  const uint64_t b_base = uniform64(
      (uint64_t)(TRANS ? p.w16 + (int64_t)kt0 * kBK * N + n0 : p.w16 + (int64_t)kt0 * kBK));
  const uint64_t b_step = TRANS ? (uint64_t)kBK * N * sizeof(f16) : (uint64_t)kBK * sizeof(f16);
  unsigned a_off[LA];
  unsigned b_off[LB];
#pragma unroll
  for (int j = 0; j < LA; ++j) {
    const int q = (j * NLW + lw) * 64 + lane;
    const int row = q >> 3, c = (q & 7) ^ swz_k(q >> 3);
    const int64_t r = m0 + row < M ? row : M - 1 - m0;   // rows past M: never stored
    a_off[j] = (unsigned)((r * p.lda + c * 8) * (int64_t)sizeof(f16));
  }
#pragma unroll
  for (int j = 0; j < LB; ++j) {
    const int q = (j * NLW + lw) * 64 + lane;
    if (!TRANS) {
      const int row = q >> 3, c = (q & 7) ^ swz_k(q >> 3);
      int64_t n = n0 + row;
      if (EPI == EPI_SWIGLU_FWD) {
        const int64_t g = n >> 6, w = n & 63;
        n = w < 32 ? g * 32 + w : p.inter + g * 32 + (w - 32);
      }
      b_off[j] = (unsigned)((n * K + c * 8) * (int64_t)sizeof(f16));
    } else {
      const int k = q / NCH, c = (q % NCH) ^ swz_n(q / NCH);
      b_off[j] = (unsigned)(((int64_t)k * N + c * 8) * (int64_t)sizeof(f16));
    }
  }
  // load d (0 .. LOADS-1) of step kt into stage st
  auto issue = [&](int kt, int st, int d) {
    if (d < LA) {
      const unsigned dst = __builtin_amdgcn_readfirstlane(
          lds_offset(As + st * SA + (d * NLW + lw) * 512));
      dma16s(a_base + (uint64_t)kt * (kBK * sizeof(f16)), a_off[d], dst);
    } else {
      const int j = d - LA;
      const unsigned dst = __builtin_amdgcn_readfirstlane(
          lds_offset(Bs + st * SB + (j * NLW + lw) * 512));
      dma16s(b_base + (uint64_t)kt * b_step, b_off[j], dst);
    }
  };

  // ---- W4: the W tile of every step dequantised from packed NF4 by the workgroup itself (no fp16
  // weight in memory).  Each thread converts PW consecutive weights of one W row per step: NT,
  // tile row tid / (64 / PW) at k offset PW (tid % (64 / PW)); NN, tile k-row tid / (BN / PW) at
  // column offset PW (tid % (BN / PW)).  PW divides a 64-weight first-level block, so one absmax
  // per piece.  Step j's packed bytes, code and second-level scale/offset are loaded during step
  // j - NST - 1, converted beside step j - NST's first sub-steps and written to stage j % NST
  // after step j - NST's barrier, where the A refill of the same stage goes out.
  constexpr int PW = BN * kBK / kThreads;   // 32 (256-wide tiles) or 16 (128-wide)
  static_assert(!W4 || PW == 32 || PW == 16, "W4 pieces");
  constexpr int PWD = PW / 8;               // packed dwords per piece = 16-byte LDS chunks
  int64_t w4_e0 = 0;                        // the piece's first element at step 0
  int w4_lds = 0;                           // its LDS offset (halves) in a stage, chunk 0
  int w4_swz = 0;
  if constexpr (W4) {
    if (!TRANS) {
      constexpr int PPR = kBK / PW;
      const int row = tid / PPR, pc = tid % PPR;
      int64_t n = n0 + row;
      if (EPI == EPI_SWIGLU_FWD) {
        const int64_t g = n >> 6, w = n & 63;
        n = w < 32 ? g * 32 + w : p.inter + g * 32 + (w - 32);
      }
      w4_e0 = n * K + (int64_t)kt0 * kBK + pc * PW;
      w4_lds = row * kBK;
      w4_swz = swz_k(row);
      w4_lds |= (pc * PWD) << 16;            // first chunk index, kept in the high half
    } else {
      constexpr int PPR = BN / PW;
      const int k = tid / PPR, pc = tid % PPR;
      w4_e0 = ((int64_t)kt0 * kBK + k) * N + n0 + pc * PW;
      w4_lds = k * BN;
      w4_swz = swz_n(k);
      w4_lds |= (pc * PWD) << 16;
    }
  }
  struct W4Piece {
    uint32_t w[PWD];
    uint32_t qa;
    float s2, o2;
  };
  auto w4_load = [&](int kt) {
    W4Piece r;
    const int64_t e = w4_e0 + (TRANS ? (int64_t)kt * kBK * N : (int64_t)kt * kBK);
    if constexpr (PWD == 4) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(p.packed + (e >> 1));
#pragma unroll
      for (int i = 0; i < 4; ++i) r.w[i] = v[i];
    } else {
      const u32x2 v = *reinterpret_cast<const u32x2*>(p.packed + (e >> 1));
#pragma unroll
      for (int i = 0; i < PWD; ++i) r.w[i] = v[i];
    }
    r.qa = p.qabs[e >> 6];
    r.s2 = p.scale2[e >> 14];
    r.o2 = p.offset2[e >> 14];
    return r;
  };
  u32x4 w4_out[PWD];   // the converted piece: PWD chunks of 8 fp16
  auto w4_convert = [&](const W4Piece& r) {
    const float* lut = w4tab;
    const float* c2 = w4tab + 16;
    const float amax = dk_absmax(c2[r.qa & 0xffu], r.s2, r.o2);
#pragma unroll
    for (int i = 0; i < PWD; ++i) w4_out[i] = dk_dequant_word(r.w[i], amax, lut);
  };
  auto w4_write = [&](int st) {
    const int c0 = w4_lds >> 16;
#pragma unroll
    for (int i = 0; i < PWD; ++i)
      *reinterpret_cast<u32x4*>(Bs + st * SB + (w4_lds & 0xffff) + (((c0 + i) ^ w4_swz) * 8)) =
          w4_out[i];
  };

  // wait until at most `later` steps of this lane's loads are still in flight
  auto wait_loads = [&](int later) {
    if (NST > 3 && later >= 3) wait_vmem<3 * LOADS>();
    else if (NST > 2 && later >= 2) wait_vmem<2 * LOADS>();
    else if (later >= 1) wait_vmem<LOADS>();
    else wait_vmem<0>();
  };
  // W4, before a step's barrier: every A refill issued so far has landed; only the packed loads
  // of the current step (the 4 newest vector-memory instructions, issued after them) may still
  // be in flight
  constexpr int kW4Loads = 4;

  // ---- main loop.  Step kt lives in stage kt % NST.  In step kt: sub-step 0's MFMAs run beside
  // the operand reads of sub-step 1; then wait for this wave's loads of step kt + 1 and for every
  // wave's last read of stage kt % NST (one barrier), refill that stage with step kt + NST,
  // spreading the DMA instructions between sub-step 1's MFMAs, which run beside the first reads of
  // step kt + 1.
  if constexpr (SPEC) {
    if (loader) {
      // the loading waves: the same loads, waits and barriers as below, no MFMAs; the refill
      // of each stage goes out right after the barrier that frees it
#pragma unroll
      for (int q = 0; q < NST; ++q)
        if (q < nk)
#pragma unroll
          for (int d = 0; d < LOADS; ++d) issue(q, q, d);
      wait_loads((nk < NST ? nk : NST) - 1);
      __syncthreads();
      for (int kt = 0; kt < nk; ++kt) {
        wait_loads((nk - 1 < kt + NST - 1 ? nk - 1 : kt + NST - 1) - (kt + 1));
        __syncthreads();
        if (kt + NST < nk)
#pragma unroll
          for (int d = 0; d < LOADS; ++d) issue(kt + NST, kt & (NST - 1), d);
      }
      // the second 32-row strip of computing wave w - NCW, handed over through LDS (below), and
      // its epilogue: every wave finishes one 32 x 64 strip, as in the 8-wave 128 x 128 tile
      __syncthreads();
      const int c = wave - NCW;
      f32x16 strip[1][TN];
      const float* hand = reinterpret_cast<const float*>(Bs) + c * (kEpiScratch / 4);
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) strip[0][j][v] = hand[(j * 16 + v) * 64 + lane];
      wave_epilogue<TRANS, EPI, 1, TN>(
          p, strip, m0 + (c / WAVES_N) * WM + 32, n0 + (c % WAVES_N) * WN,
          reinterpret_cast<uint8_t*>(Bs) + c * kEpiScratch,
          reinterpret_cast<const uint8_t*>(Bs) + (c ^ 1) * kEpiScratch);
      return;
    }
  }
  W4Piece w4_next;   // W4: the packed piece of step kt + NST (loaded one step before its use)
  if constexpr (W4) {
    // the first NST steps' W tiles converted and written before the loop (their loads waited at
    // once: a prologue)
#pragma unroll
    for (int q = 0; q < NST; ++q)
      if (q < nk) {
        w4_convert(w4_load(q));
        w4_write(q);
      }
    w4_next = w4_load(NST < nk ? NST : nk - 1);   // clamped: its result is then never written
  }
  if (!SPEC) {
#pragma unroll
    for (int q = 0; q < NST; ++q)
      if (q < nk)
#pragma unroll
        for (int d = 0; d < LOADS; ++d) issue(q, q, d);
    if (W4) wait_vmem<0>();
    else wait_loads((nk < NST ? nk : NST) - 1);
  }
  __syncthreads();
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;   // this wave's block of the tile
  f32x16 acc[TM][TN];
  // ---- MFMA operands: v_mfma_f32_16x16x32_f16 on 16 x 16 blocks (TM16 x TN16 per wave), two
  // 32-wide sub-steps per 64-wide step.  A operand of lane l: row l % 16 of a 16-row block, k
  // 8 (l / 16) .. + 7 of the sub-step; W likewise by column.  (Measured on MI355X, a loop of the
  // GEMM's protocol on random fp16 operands: 1.40 against 1.28-1.29 PFLOP/s with
  // v_mfma_f32_32x32x16_f16 on 32 x 32 blocks; the clock, which power sets, 1.77 against
  // 1.51 GHz: the smaller MFMA spends less energy per FLOP.  In the step every GEMM's share of
  // the power budget counts: the 128 x 128 tiles on it too measured slower replayed alone but
  // 14.05 -> 13.65 ms per step.)
  constexpr int TM16 = 2 * TM, TN16 = 2 * TN;
  const int r16 = lane & 15;
  const int hx = swz_k(r16);
  int fo[2];   // operand offset of each 32-wide sub-step
#pragma unroll
  for (int q = 0; q < 2; ++q) fo[q] = r16 * kBK + ((4 * q + (lane >> 4)) ^ hx) * 8;
  // NN: the 16-lane group g reads rows 8 g + 4 h .. + 3 of the sub-step (h = 0, 1) transposed
  const int tr_k = 8 * (lane >> 4) + (r16 >> 2);
  const int tr_n = 4 * (lane & 3);
  int nn_off[TN16];
#pragma unroll
  for (int j = 0; j < TN16; ++j) {
    const int n = wn * WN + 16 * j + tr_n;
    nn_off[j] = tr_k * BN + (((n >> 3) ^ swz_n(tr_k)) * 8) + (n & 7);
  }

  f32x4 a16[TM16][TN16];
#pragma unroll
  for (int i = 0; i < TM16; ++i)
#pragma unroll
    for (int j = 0; j < TN16; ++j) a16[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // W fragments double-buffered (the next sub-step's fragment j read after MFMA j).  A
  // fragments: with 32 MFMAs per sub-step (128 accumulator registers, no room for two buffers)
  // single-buffered, the next sub-step's fragment i read right after the last MFMA that uses
  // the current one, MFMA (i + 1) TN16 - 1 (the MFMAs go row by row), a whole sub-step before
  // its first use; with 16 or fewer, double-buffered and read after MFMA TN16 + i
  constexpr int NMFMA = TM16 * TN16;
  // MFMA k of a sub-step: A fragment k / TN16 and, row by row in a serpentine, W fragment kj(k),
  // so that two MFMAs in a row share an operand at each row change too (every accumulator still
  // takes its sub-steps in order: the sums are unchanged).  Measured on MI355X, bit-identical: the
  // large GEMMs 0.7-0.9 % faster in the step
  auto kj = [](int k) { return (k / TN16) & 1 ? TN16 - 1 - k % TN16 : k % TN16; };
  constexpr bool A2 = NMFMA <= 16;
  f16x8 fa[A2 ? 2 : 1][TM16], fb[2][TN16];
  auto read_a = [&](int st, int s, int i, int buf) {
    fa[A2 ? buf : 0][i] =
        *reinterpret_cast<const f16x8*>(As + st * SA + (wm * WM + 16 * i) * kBK + fo[s]);
  };
  auto a_slot = [](int i) {
    return A2 ? (TN16 + i < NMFMA ? TN16 + i : NMFMA - 1) : (i + 1) * TN16 - 1;
  };
  auto read_b = [&](int st, int s, int j, int buf) {
    if (!TRANS) {
      fb[buf][j] = *reinterpret_cast<const f16x8*>(Bs + st * SB + (wn * WN + 16 * j) * kBK + fo[s]);
    } else {
      // ds_read_b64_tr_b16: each 16-lane group reads 4 rows x 16 columns (lane i of the group
      // addressing row i / 4, columns 4 (i % 4) .. + 3); lane i receives column i's 4 values
      const f16* q = Bs + st * SB + 32 * s * BN + nn_off[j];
      const f16x4 lo = read_tr(q), hi = read_tr(q + 4 * BN);
      fb[buf][j] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  };
  // the reads that go out after MFMA k of a sub-step (those of sub-step s of stage st, into
  // buffer buf)
  auto reads_after = [&](int k, int st, int s, int buf) {
#pragma unroll
    for (int j = 0; j < TN16; ++j)
      if (j == k) read_b(st, s, j, buf);
#pragma unroll
    for (int i = 0; i < TM16; ++i)
      if (a_slot(i) == k) read_a(st, s, i, buf);
  };
  static_assert(TN16 <= NMFMA, "W fragment reads beside the MFMAs");
  // scheduling: MFMA k, then the DS reads placed after it (the other instructions, such as the W4
  // conversion, free to fill in)
  auto mfma_group = [&](int k) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    int n = 0;
#pragma unroll
    for (int j = 0; j < TN16; ++j)
      if (j == k) n += TRANS ? 2 : 1;
#pragma unroll
    for (int i = 0; i < TM16; ++i)
      if (a_slot(i) == k) n += 1;
    if (n == 1) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    else if (n == 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    else if (n == 3) __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
  };

#pragma unroll
  for (int i = 0; i < TM16; ++i) read_a(0, 0, i, 0);
#pragma unroll
  for (int j = 0; j < TN16; ++j) read_b(0, 0, j, 0);
  for (int kt = 0; kt < nk; ++kt) {
    const int st = kt & (NST - 1);
    W4Piece w4_after;
    if constexpr (W4) {
      // step kt + NST + 1's packed piece (clamped at the end: loaded, never written)
      w4_after = w4_load(kt + NST + 1 < nk ? kt + NST + 1 : nk - 1);
    }
    if (W4) w4_convert(w4_next);   // step kt + NST's W tile, beside the MFMAs
    // sub-step 0 (W buffer 0), beside the reads of sub-step 1
#pragma unroll
    for (int k = 0; k < NMFMA; ++k) {
      a16[k / TN16][kj(k)] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          fa[0][k / TN16], fb[0][kj(k)], a16[k / TN16][kj(k)], 0, 0, 0);
      reads_after(k, st, 1, 1);
    }
#pragma unroll
    for (int k = 0; k < NMFMA; ++k) mfma_group(k);
    // steps issued after kt + 1 that may still be in flight: min(nk - 1, kt + NST - 1) - (kt + 1)
    if (W4) wait_vmem<kW4Loads>();
    else if (!SPEC) wait_loads((nk - 1 < kt + NST - 1 ? nk - 1 : kt + NST - 1) - (kt + 1));
    __syncthreads();
    const bool more = kt + 1 < nk;
    const int st1 = (kt + 1) & (NST - 1);
    const bool refill = !SPEC && kt + NST < nk;
    if constexpr (W4) {
      if (refill) w4_write(st);
      w4_next = w4_after;
    }
    // sub-step 1 (W buffer 1), which issues the refill and reads step kt + 1's first operands, at
    // wave priority 1: the wave past the barrier gets its DMA out ahead of the other wave's
    // operand reads (measured on MI355X: every GEMM of the step 0.5-6 % faster, the step ~1 %)
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int k = 0; k < NMFMA; ++k) {
      a16[k / TN16][kj(k)] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          fa[A2 ? 1 : 0][k / TN16], fb[1][kj(k)], a16[k / TN16][kj(k)], 0, 0, 0);
      if (more) reads_after(k, st1, 0, 0);
#pragma unroll
      for (int d = k * LOADS / NMFMA; d < (k + 1) * LOADS / NMFMA; ++d)
        if (refill) issue(kt + NST, st, d);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_setprio(0);
  }
  // the 16 x 16 results as 32 x 32 blocks (register 4 (2 a + b) + r of block (i, j): register r
  // of 16 x 16 block (2 i + a, 2 j + b)), the layout the epilogue takes
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = a16[2 * i + (v >> 3)][2 * j + ((v >> 2) & 1)][v & 3];
  // every wave is past the last barrier, after which no wave reads a stage and no load is in
  // flight: the stages are free for the per-wave epilogue scratch

  if constexpr (SPEC) {
    // (128 x 128 tiles have no split K.)  The first 32-row strip is finished here, the second by
    // loading wave w + NCW: handed over in its epilogue scratch slot (which it reads before it
    // writes there), lane-major so that the 64 lanes of each store and load are contiguous
    static_assert(TM == 2, "two 32-row strips per computing wave");
    float* hand = reinterpret_cast<float*>(Bs) + wave * (kEpiScratch / 4);
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) hand[(j * 16 + v) * 64 + lane] = acc[1][j][v];
    __syncthreads();
    f32x16 strip[1][TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) strip[0][j] = acc[0][j];
    wave_epilogue<TRANS, EPI, 1, TN>(p, strip, m0 + wm * WM, n0 + wn * WN,
                                     reinterpret_cast<uint8_t*>(As) + wave * kEpiScratch,
                                     reinterpret_cast<const uint8_t*>(As) + (wave ^ 1) * kEpiScratch);
    return;
  }
  if (part) {
    // split-K: this wave's fp32 partial blocks; in a block, registers 4 q .. 4 q + 3 of lane l
    // at 256 q + 4 l, so each 16-byte store instruction writes 1 KiB contiguous; the reduce
    // launch sums the splits and runs the epilogue
    float* mine = part + (int64_t)wave * TM * TN * 1024 + 4 * lane;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          *reinterpret_cast<f32x4*>(mine + (i * TN + j) * 1024 + 256 * q) =
              f32x4{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
    return;
  }
  // the epilogue scratch: 16 KB per wave, waves 0-3 in the A stages, 4-7 in the W stages
  uint8_t* escr = reinterpret_cast<uint8_t*>(wave < 4 ? As : Bs) + (wave & 3) * kEpiScratch;
  // the partner wave: the other 64-column half of the same rows (rotary epilogue)
  const int pw = wave ^ 1;
  const uint8_t* pscr = reinterpret_cast<const uint8_t*>(pw < 4 ? As : Bs) + (pw & 3) * kEpiScratch;
  static_assert(WAVES_N % 2 == 0, "partner waves share rows");
  wave_epilogue<TRANS, EPI, TM, TN>(p, acc, m0 + wm * WM, n0 + wn * WN, escr, pscr);
}

// main_tiles workgroups run 256 x 256 tiles and tail_wgs run the tiles past main_tiles as
// 128 x 128 quarters: the full tiles first, except in the SwiGLU backward, whose quarters go
// first.  There that staggers the rounds: the CUs that ran a quarter start their full tiles
// later than the rest, so the rounds' epilogues (HBM-bound: they read and rewrite [g|u]) do not
// all fall at once (measured on MI355X: 79.7 -> 77.2 us at M = 2048).  Elsewhere the stagger
// leaves the time unchanged but, with the XCDs' tiles no longer in step along K, fetches more
// (gate|up forward 198 -> 287 MB).  With split-K (p.splits > 1, LINEAR only) full-tile
// workgroup b (counted from the first) runs split b / tiles of tile b % tiles and stores its
// fp32 partial tile at p.part[tile][split].  Tiles are numbered M-fastest.  The p.sums.wgs
// workgroups after the tiles (NN LINEAR) run the LoRA column sums the launch carries, the
// p.side.wgs after those its dequant work; dispatched last, they take the CUs the tiles leave
// idle.  persist (fp16 SwiGLU GEMMs over more than one round): the grid is one workgroup per CU,
// gridDim.x / 8 per XCD, and each walks its XCD's share of the same tiles in the same order
// (full tiles then quarters, or quarters first in the backward), so that a tile's first loads go
// out while the previous tile's epilogue stores drain (measured on MI355X at M = 2048: gate|up
// forward 111.7-112.0 -> 110.5 us, step -0.05 ms; down^T backward 75.0 -> 74.7 us, step
// -0.03 ms).
template <bool TRANS, int EPI, bool W4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void hgemm_kernel(GemmParams p, int main_tiles, int tail_wgs, int persist) {
  __shared__ __attribute__((aligned(1024))) f16 As[kStages * kStageHalves];
  __shared__ __attribute__((aligned(1024))) f16 Bs[kStages * kStageHalves];
  // W4: the 16 NF4 values and the 256-entry second-level code table
  __shared__ float w4tab[W4 ? 16 + 256 : 1];
  static_assert(side_dequant_lds <= kStages * kStageHalves * 2 && kSideThreads == kThreads,
                "side dequant in the kernel's LDS");
  static_assert(colsum_lds_bytes<16>() <= kStages * kStageHalves * 2 && kSumThreads == kThreads,
                "carried LoRA column sums in the kernel's LDS");
  if constexpr ((EPI == EPI_SWIGLU_FWD || EPI == EPI_SWIGLU_BWD) && !W4) {
    if (persist) {
      // workgroup x + 8 r of XCD x takes that XCD's full tiles r, r + per, ... (numbered as
      // below: XCD x owns the contiguous run [x nf8, (x + 1) nf8)) and its quarters r, r + per,
      // ... (quarter index 8 qi + x, as below), the quarters first in the SwiGLU backward
      const int x = blockIdx.x & 7, r = blockIdx.x >> 3, per = (int)gridDim.x >> 3;
      const int nf8 = main_tiles >> 3, nq8 = tail_wgs >> 3;
      const int nk = (int)(p.K / kBK);
      bool first = true;
      auto quarters = [&]() {
        for (int qi = r; qi < nq8; qi += per) {
          if (!first) __syncthreads();   // every wave is done with the previous tile's LDS
          first = false;
          int64_t m0, n0;
          if (p.xcd_gm) {
            const int gm = p.xcd_gm;
            const int bm = p.tiles_m / gm, bn = (tail_wgs / 4 / p.tiles_m) / (8 / gm);
            const int qm = qi % (2 * bm), qn = qi / (2 * bm);
            m0 = (int64_t)((x % gm) * bm) * kTile + 128 * qm;
            n0 = (int64_t)(main_tiles / p.tiles_m + (x / gm) * bn) * kTile + 128 * qn;
          } else {
            const int u = x * nq8 + qi;
            const int parent = main_tiles + u / 4, quarter = u % 4;
            m0 = (int64_t)(parent % p.tiles_m) * kTile + 128 * (quarter & 1);
            n0 = (int64_t)(parent / p.tiles_m) * kTile + 128 * (quarter >> 1);
          }
          if (m0 < p.M)
            gemm_tile<TRANS, EPI, 128, 128, W4 || TRANS ? 4 : 2, 4, W4>(p, m0, n0, 0, nk, nullptr, As, Bs, w4tab);
        }
      };
      if (EPI == EPI_SWIGLU_BWD) quarters();
      for (int fi = r; fi < nf8; fi += per) {
        if (!first) __syncthreads();
        first = false;
        const int tile = x * nf8 + fi;
        gemm_tile<TRANS, EPI, 256, 256, 2, 2, W4>(p, (int64_t)(tile % p.tiles_m) * kTile,
                                                  (int64_t)(tile / p.tiles_m) * kTile, 0, nk,
                                                  nullptr, As, Bs, w4tab);
      }
      if (EPI == EPI_SWIGLU_FWD) quarters();
      return;
    }
  }
  if ((int)blockIdx.x >= main_tiles + tail_wgs) {
    int j = (int)blockIdx.x - main_tiles - tail_wgs;
    if constexpr (TRANS && EPI == EPI_LINEAR) {
      if (j < p.sums.wgs) {
        colsum_run<16>(p.sums.jobs, p.sums.rows,
                       colsum_block_of(j, p.sums.wgs, main_tiles + tail_wgs),
                       reinterpret_cast<uint8_t*>(As));
        return;
      }
      j -= p.sums.wgs;
    }
    side_dequant(p.side, j, reinterpret_cast<uint8_t*>(As));
    return;
  }
  const int nk_all = (int)(p.K / kBK);
  if constexpr (W4) {
    if (threadIdx.x < 16) w4tab[threadIdx.x] = p.nf4[threadIdx.x];
    if (threadIdx.x < 256) w4tab[16 + threadIdx.x] = p.code2[threadIdx.x];
    __syncthreads();
  }
  constexpr bool kQuartersFirst = EPI == EPI_SWIGLU_BWD;
  const int fbase = kQuartersFirst ? tail_wgs : 0;    // first full-tile workgroup
  const int qbase = kQuartersFirst ? 0 : main_tiles;  // first quarter workgroup
  int b = blockIdx.x;
  if (b >= fbase && b < fbase + main_tiles) {
    // workgroups are dealt to the 8 XCDs round-robin (workgroup i to XCD i % 8): give each XCD a
    // contiguous run of tiles.  XCD x's full-tile workgroups are first, first + 8, ... from the
    // first index at or past fbase that it receives.
    if ((main_tiles & 7) == 0) {
      const int x = b & 7, first = fbase + ((x - fbase) & 7);
      b = x * (main_tiles >> 3) + ((b - first) >> 3);
    } else {
      b -= fbase;
    }
    // split-K: the splits are the slowest index, so an XCD's run covers neighbouring tiles of
    // one K range, which share A and W slices in its L2
    const int tiles = main_tiles / p.splits;
    const int tile = b % tiles, split = b / tiles;
    const int64_t m0 = (int64_t)(tile % p.tiles_m) * kTile;
    const int64_t n0 = (int64_t)(tile / p.tiles_m) * kTile;
    const int kt0 = (int)((int64_t)nk_all * split / p.splits);
    const int nk = (int)((int64_t)nk_all * (split + 1) / p.splits) - kt0;
    float* part =
        p.splits > 1 ? p.part + ((int64_t)tile * p.splits + split) * kTile * kTile : nullptr;
    gemm_tile<TRANS, EPI, 256, 256, 2, 2, W4>(p, m0, n0, kt0, nk, part, As, Bs, w4tab);
  } else {
    int64_t m0, n0;
    const int t = b - qbase;
    if (p.xcd_gm) {
      // the quarters' parent tiles form a grid of tiles_m rows by the columns past the full tiles;
      // XCD x = t % 8 (workgroups are dealt to the XCDs round-robin) takes block (x % gm, x / gm)
      // of a gm x (8 / gm) split of that grid, so that its L2 holds the A rows and W rows of its
      // block only (the hplan choice of gm minimises them), and walks the block's quarters
      // M-fastest
      const int gm = p.xcd_gm, x = t & 7, r = t >> 3;
      const int bm = p.tiles_m / gm, bn = (tail_wgs / 4 / p.tiles_m) / (8 / gm);
      const int qm = r % (2 * bm), qn = r / (2 * bm);
      m0 = (int64_t)((x % gm) * bm) * kTile + 128 * qm;
      n0 = (int64_t)(main_tiles / p.tiles_m + (x / gm) * bn) * kTile + 128 * qn;
    } else {
      int u = t;
      if ((tail_wgs & 7) == 0 && (qbase & 7) == 0) u = (u & 7) * (tail_wgs >> 3) + (u >> 3);
      const int parent = main_tiles + u / 4, quarter = u % 4;
      m0 = (int64_t)(parent % p.tiles_m) * kTile + 128 * (quarter & 1);
      n0 = (int64_t)(parent / p.tiles_m) * kTile + 128 * (quarter >> 1);
    }
    if (m0 >= p.M) return;
    gemm_tile<TRANS, EPI, 128, 128, W4 || TRANS ? 4 : 2, 4, W4>(p, m0, n0, 0, nk_all, nullptr, As, Bs, w4tab);
  }
}

// Split-K, second launch: one wave per 32 x 32 block of a 256 x 256 tile (64 per tile) sums the
// block's split partials in split order (fixed, so the result is deterministic) and runs the
// epilogue on it.  The kernel boundary orders it after every partial store.
template <bool TRANS, int EPI>
__global__ __launch_bounds__(64) void hgemm_reduce_kernel(GemmParams p) {
  // 8 KB of LDS per one-wave workgroup, so that 20 of them fit a CU
  __shared__ __attribute__((aligned(16))) uint8_t escr[epi_scratch_bytes(1)];
  constexpr int TM = 4, TN = 2;   // the blocks of one 128 x 64 wave block of the first launch
  const int lane = threadIdx.x;
  const int tile = blockIdx.x / 64, blk = blockIdx.x % 64;
  const int wave = blk / (TM * TN), i = (blk / TN) % TM, j = blk % TN;
  const int64_t m0 = (int64_t)(tile % p.tiles_m) * kTile + (wave / 4) * 128 + 32 * i;
  const int64_t n0 = (int64_t)(tile / p.tiles_m) * kTile + (wave % 4) * 64 + 32 * j;
  if (m0 >= p.M) return;
  const float* src = p.part + (int64_t)tile * p.splits * kTile * kTile +
                     (wave * TM * TN + i * TN + j) * 1024 + 4 * lane;
  f32x16 acc[1][1];
  f32x4 v_all[4][4];
  // four splits' loads in flight at a time (clamped, straight-line), then their sum in split order
  for (int sp = 0; sp < p.splits; sp += 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int s = sp + u < p.splits ? sp + u : p.splits - 1;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v_all[u][q] = *reinterpret_cast<const f32x4*>(src + (int64_t)s * kTile * kTile + 256 * q);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (sp + u < p.splits)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          acc[0][0][v] = sp + u == 0 ? v_all[u][v >> 2][v & 3] : acc[0][0][v] + v_all[u][v >> 2][v & 3];
  }
  wave_epilogue<TRANS, EPI, 1, 1>(p, acc, m0, n0, escr, escr);   // never rotary: no split-K
}

int cu_count() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  if (!cached[dev]) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cached[dev] = n;
  }
  return cached[dev];
}

// The launch shape of a GEMM on this kernel, or ok = false.
struct HPlan {
  bool ok;
  int64_t tiles_m, tiles_n, main_wgs, tail_wgs;
  int splits;
  int xcd_gm;   // GemmParams::xcd_gm
};

// The split of the quarters' parent grid (tiles_m rows by the tail's columns) into one block per
// XCD, gm blocks along M by 8 / gm along N, that minimises the rows of A plus rows of W one XCD
// reads (bm + bn tiles); 0 when no split divides the grid (then runs of quarters per XCD).
int xcd_blocks(int64_t tiles_m, int64_t main_wgs, int64_t tail_wgs, int qbase) {
  if (tail_wgs <= 0 || tail_wgs % 32 || qbase % 8 || main_wgs % tiles_m) return 0;
  const int64_t parents = tail_wgs / 4;
  if (parents % tiles_m) return 0;
  const int64_t cols = parents / tiles_m;
  int best = 0;
  int64_t cost = 0;
  for (int gm = 1; gm <= 8; gm *= 2) {
    const int gn = 8 / gm;
    if (tiles_m % gm || cols % gn) continue;
    const int64_t c = tiles_m / gm + cols / gn;
    if (!best || c < cost) {
      best = gm;
      cost = c;
    }
  }
  return best;
}

HPlan hplan_tiles(int64_t M, int64_t N, int64_t K, int epi, bool no_split, bool nt) {
  HPlan h{false, 0, 0, 0, 0, 1, 0};
  if (M <= 0 || N % kTile || K % kBK || K < kBK) return h;
  const int cus = cu_count();
  if (cus <= 0) return h;
  h.tiles_m = (M + kTile - 1) / kTile;
  h.tiles_n = N / kTile;
  const int64_t tiles = h.tiles_m * h.tiles_n;
  if (tiles * 4 > 0x7fffffff) return h;
  if (tiles >= cus) {
    // a last round at most half full runs as 128 x 128 quarters
    h.main_wgs = tiles;
    const int64_t rest = tiles % cus;
    if (rest > 0 && rest <= cus / 2) {
      h.main_wgs = tiles - rest;
      h.tail_wgs = 4 * rest;
    }
    h.ok = true;
    return h;
  }
  // fewer tiles than CUs: split K so that the splits fill the CUs once.  The fp32 partials cost
  // two passes over splits x tiles x 256 KB, which only long K (4096 or more) repays; LINEAR
  // only, at least 4 row tiles.  NT GEMMs whose 128 x 128 quarters fill half the CUs run as
  // quarters over the whole K instead: their loop (computing and loading waves apart) does as
  // much per CU as the full tiles' in the step, without the partials' round trip or the reduce
  // launch (down forward at M = 2048, K = 8960: 71.8 -> 61.8 us in the step)
  const int64_t quarters = (M + 127) / 128 * (N / 128);
  if (!no_split && epi == EPI_LINEAR && h.tiles_m >= 4 && K >= 4096 &&
      !(nt && quarters * 2 >= cus)) {
    int64_t s = cus / tiles;
    if (s > K / kBK / 8) s = K / kBK / 8;
    if (s >= 2) {
      h.splits = (int)s;
      h.main_wgs = tiles * s;
      h.ok = true;
      return h;
    }
  }
  // otherwise every tile as 128 x 128 quarters, when they fill at least half the CUs
  if (quarters * 2 < cus && !no_split) return h;
  h.main_wgs = 0;
  h.tail_wgs = 4 * tiles;
  h.ok = true;
  return h;
}

HPlan hplan(int64_t M, int64_t N, int64_t K, int epi, bool no_split, bool nt) {
  HPlan h = hplan_tiles(M, N, K, epi, no_split, nt);
  if (h.ok && h.splits == 1)
    h.xcd_gm = xcd_blocks(h.tiles_m, h.main_wgs, h.tail_wgs,
                          epi == EPI_SWIGLU_BWD ? 0 : (int)h.main_wgs);
  return h;
}

}  // namespace

int64_t hgemm_workspace(int64_t M, int64_t N, int64_t K, int epi, bool nt) {
  const HPlan h = hplan(M, N, K, epi, false, nt);
  if (!h.ok) return -1;
  if (h.splits == 1) return 0;
  return h.main_wgs * kTile * kTile * (int64_t)sizeof(float);
}

// The epilogue writes 16-byte vectors of 8 consecutive columns.
static bool vector_outputs_ok(const GemmParams& p, int epi) {
  if (epi == EPI_LINEAR)
    return dk_aligned(p.out, 16) && p.ldo % (p.out_mode == DK_OUT_F16 ? 8 : 4) == 0;
  if (epi == EPI_SWIGLU_FWD)
    return dk_aligned(p.out, 16) && p.ldo % 8 == 0 && (!p.gu || dk_aligned(p.gu, 16)) &&
           p.inter % 8 == 0;
  return dk_aligned(p.gu, 16) && p.inter % 8 == 0;
}

template <bool TRANS, int EPI, bool W4>
int hgemm_launch(const GemmParams& p0, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (!(W4 ? p0.packed && p0.qabs && p0.scale2 && p0.offset2 && p0.code2 && p0.nf4 &&
                 dk_aligned(p0.packed, 16)
           : p0.w16 != nullptr) ||
      !vector_outputs_ok(p0, EPI))
    return kHgemmDeclined;
  // the rotary epilogue pairs the two column halves of a head inside one workgroup: no split-K,
  // and 128-column tiles at any size
  const bool rope = p0.rope_pos != nullptr;
  if (rope && (TRANS || EPI != EPI_LINEAR)) return kHgemmDeclined;
  // the loads' 32-bit byte offsets: A within a 256-row tile, W (NT) within the whole weight
  // (the SwiGLU pairing reaches its last row), W (NN) within 64 rows of a step
  constexpr int64_t kOffMax = (int64_t)1 << 32;
  if ((kTile * p0.lda + p0.K) * (int64_t)sizeof(f16) >= kOffMax ||
      (!W4 && (TRANS ? (int64_t)kBK * p0.N : p0.N * p0.K) * (int64_t)sizeof(f16) >= kOffMax))
    return kHgemmDeclined;
  const HPlan h = hplan(p0.M, p0.N, p0.K, EPI, rope, !TRANS);
  if (!h.ok) return kHgemmDeclined;
  GemmParams p = p0;
  p.tiles_m = (int)h.tiles_m;
  p.tiles_n = (int)h.tiles_n;
  p.splits = h.splits;
  p.xcd_gm = h.xcd_gm;
  if (h.splits > 1) {
    // the partials go to the caller's workspace; without room for them, decline
    if (!ws || ws_bytes < h.main_wgs * kTile * kTile * (int64_t)sizeof(float) || !dk_aligned(ws, 256))
      return kHgemmDeclined;
    p.part = reinterpret_cast<float*>(ws);
  }
  // carried dequant: the given workgroup count, or (auto) the CUs the last round leaves idle
  int side = 0;
  if (p.side.sb1 > p.side.sb0 && p.side.wgs != 0) {
    side = p.side.wgs;
    if (side < 0) {
      const int rest = (int)((h.main_wgs + h.tail_wgs) % cu_count());
      side = rest ? cu_count() - rest : 0;
      if (side < 16) side = 16;
    }
    p.side.wgs = side;
  }
  // carried LoRA column sums (NN LINEAR only; the caller sets p.sums.wgs)
  const int sums = TRANS && EPI == EPI_LINEAR ? p.sums.wgs : 0;
  p.sums.wgs = sums;
  // the fp16 SwiGLU GEMMs that take more than one round run one persistent workgroup per CU
  // when their tiles divide evenly over the XCDs' CUs
  const int cus = cu_count();
  const int persist = ((EPI == EPI_SWIGLU_FWD && h.main_wgs > cus) ||
                       (EPI == EPI_SWIGLU_BWD && h.tail_wgs > 0)) && !W4 && h.splits == 1 &&
                      side == 0 && cus % 8 == 0 && h.main_wgs % 8 == 0 &&
                      (h.main_wgs / 8) % (cus / 8) == 0 && h.tail_wgs % 8 == 0 &&
                      h.tail_wgs / 8 <= cus / 8;
  hipLaunchKernelGGL((hgemm_kernel<TRANS, EPI, W4>),
                     dim3((unsigned)(persist ? cus : h.main_wgs + h.tail_wgs + sums + side)),
                     dim3(kThreads), 0, stream, p, (int)h.main_wgs, (int)h.tail_wgs, persist);
  DK_CHECK_LAUNCH();
  if constexpr (EPI == EPI_LINEAR) {   // hplan splits K for the LINEAR epilogue only
    if (h.splits > 1) {
      hipLaunchKernelGGL((hgemm_reduce_kernel<TRANS, EPI>),
                         dim3((unsigned)(h.tiles_m * h.tiles_n * 64)), dim3(64), 0, stream, p);
      DK_CHECK_LAUNCH();
    }
  }
  return 0;
}

template int hgemm_launch<false, EPI_LINEAR, false>(const GemmParams&, void*, int64_t, hipStream_t);
template int hgemm_launch<true, EPI_LINEAR, false>(const GemmParams&, void*, int64_t, hipStream_t);
template int hgemm_launch<false, EPI_SWIGLU_FWD, false>(const GemmParams&, void*, int64_t, hipStream_t);
template int hgemm_launch<true, EPI_SWIGLU_BWD, false>(const GemmParams&, void*, int64_t, hipStream_t);
template int hgemm_launch<false, EPI_LINEAR, true>(const GemmParams&, void*, int64_t, hipStream_t);
template int hgemm_launch<true, EPI_LINEAR, true>(const GemmParams&, void*, int64_t, hipStream_t);
template int hgemm_launch<false, EPI_SWIGLU_FWD, true>(const GemmParams&, void*, int64_t, hipStream_t);
template int hgemm_launch<true, EPI_SWIGLU_BWD, true>(const GemmParams&, void*, int64_t, hipStream_t);

}  // namespace dk
