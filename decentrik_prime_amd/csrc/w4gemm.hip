// Fused NF4 (W4) GEMMs on gfx950: dequant in LDS, v_mfma_f32_32x32x16_f16, fp32 accumulate.
//
//   forward  "NT":  C[m][n] = sum_k A[m][k] * W[n][k]      W stored [N][K], K contiguous
//   backward "NN":  C[m][n] = sum_k A[m][k] * W[k][n]      W stored [K][N], N contiguous
//
// A is fp16 row-major [M][K] (X or dY).  A workgroup owns a BM x BN tile of C and walks K in
// steps of 64.  It has 8 waves in two roles (warp specialisation):
//   - 4 consumer waves (2 x 2, each a (BM/2) x (BN/2) sub-tile) only read MFMA fragments from LDS
//     and issue MFMAs;
//   - 4 producer waves load the A tile and the packed W tile from global memory three steps
//     ahead (three register stages), look the NF4 values up in an LDS table one step ahead, and
//     write the A tile and the dequantised W tile into the LDS buffer of the next step.
// Each SIMD holds one consumer and one producer wave, so the producer's VALU dequant issues while
// the consumer's MFMAs run.  Two LDS buffers; one barrier per step.  The producers read W as
// 16-byte chunks of packed nibbles (32 consecutive weights of a stored row, inside one
// first-level block, so one absmax each) and write the dequantised chunk in its stored order:
//   NT  the W tile is K-contiguous rows padded to 72 halves, like the A tile, so every MFMA
//       operand is one ds_read_b128;
//   NN  the W tile is N-contiguous rows (stored order) padded by 16 halves; the consumers build
//       each K-contiguous operand from two ds_read_b64_tr_b16 (gfx950 transposing LDS reads).
//
// Epilogues (fused, per output element, rounding like the reference's separate ops):
//   LINEAR      y = fp16(acc + bias); + LoRA: fp16(fp32(y) + s * fp32(fp16(z B^T)))     (forward)
//               dX = fp32(fp16(acc)) + (mask ? fp32(fp16(dz A)) * keep_scale : 0)        (backward)
//               the rank-16 LoRA product is one extra MFMA per 32 x 32 tile and rank slice.
//   SWIGLU_FWD  the B rows of each consumer wave's 64 columns are 32 gate rows and the matching
//               32 up rows, so g and u of one output sit in the same lane and register:
//               act = fp16(silu(fp16(g)) * fp16(u)), optional [g | u] store.
//   SWIGLU_BWD  dact = fp16(acc), then the gated-SiLU backward in place on gu.
// Split-K (shapes with too few tiles): a first launch stores fp32 partial tiles, a second launch
// (the REDUCE instance: consumer waves only, no LDS) sums them in split order and runs the
// epilogue.
#include <mutex>

#include "gemm_common.h"

using namespace dk;

namespace {

constexpr int kBK = 64;
constexpr int kStride = kBK + 8;  // halves per K-contiguous LDS row (144 bytes)
constexpr int kPadT = 16;         // NN: halves of padding per N-contiguous LDS row of the W tile
// Waves per role: consumers are WAVES_M x 2 (64-row strips), producers as many; 128-row tiles
// run 512 threads, 256-row tiles 1024.
template <int BM>
constexpr int role_threads() { return (BM / 64) * 2 * 64; }

// REDUCE: the split-K second launch (consumer waves only): sum the partials, then the epilogue.
// Every tile runs 4 waves per SIMD (two 512-thread or one 1024-thread workgroup per CU), so the
// kernel is held to 128 VGPRs.
// F16B: W is read as fp16 from p.w16 (the two-phase path) instead of NF4 sections.
template <int BM, int BN, bool TRANS, int EPI, bool REDUCE, bool F16B>
__global__ __launch_bounds__(2 * role_threads<BM>()) __attribute__((amdgpu_waves_per_eu(4)))
void w4_gemm_kernel(GemmParams p) {
  constexpr int ROLE = role_threads<BM>();         // threads per role
  constexpr int WAVES_M = BM / 64, WAVES_N = 2;    // consumer waves
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_CHUNKS = BM * kBK / 8 / ROLE;    // 16-byte A chunks per producer thread
  constexpr int BU = BN * kBK / ROLE;              // W weights per producer thread per step
  constexpr int BU_WORDS = BU / 8;                 // packed dwords per unit
  constexpr int B_LD = TRANS ? BN + kPadT : kStride;   // halves per LDS row of the W tile
  constexpr int B_HALVES = TRANS ? kBK * B_LD : BN * kStride;
  constexpr int TILE = BM * BN;
  static_assert(TM >= 1 && TN >= 1, "tile too small");
  static_assert(BU == 16 || BU == 32, "a W unit is 16 or 32 weights of one stored row");
  static_assert(A_CHUNKS >= 1 && BM * kBK / 8 == A_CHUNKS * ROLE, "A tile split");
  static_assert(EPI != EPI_SWIGLU_FWD || (TN == 2 && !TRANS), "SwiGLU forward needs WN = 64");

  __shared__ __attribute__((aligned(16))) f16 As[2][BM * kStride];
  __shared__ __attribute__((aligned(16))) f16 Bs[2][B_HALVES];
  // byte -> (NF4[high nibble], NF4[low nibble]): one 8-byte lookup dequantises two weights
  __shared__ f32x2 pair_lut[256];
  __shared__ float c2t[256];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const bool producer = wave >= ROLE / 64;   // wave-uniform

  // XCD-aware tile order: workgroups are dealt to the 8 XCDs round-robin, so give each XCD a
  // contiguous run of tiles.  Packed W (one phase): column tiles fastest, so an XCD keeps one band
  // of A rows in its L2 while the packed W tiles (a quarter of the bytes per row) stream past it.
  // fp16 W (two phase): row tiles fastest (see launch).  With split-K the splits of one tile are
  // consecutive, so they share an XCD and its L2.
  int b = blockIdx.x;
  const int nb = gridDim.x;
  if ((nb & 7) == 0) b = (b & 7) * (nb >> 3) + (b >> 3);
  // first launch: the splits of a tile are consecutive; REDUCE: one workgroup per 32 x 32 block
  // index of the consumer sub-tiles, so the partial sums are read by TM * TN times more waves
  const int per_tile = REDUCE ? TM * TN : p.splits;
  const int split = REDUCE ? 0 : b % per_tile;
  const int tile = b / per_tile;
  const int64_t m0 = (int64_t)(p.m_fastest ? tile % p.tiles_m : tile / p.tiles_n) * BM;
  const int64_t n0 = (int64_t)(p.m_fastest ? tile / p.tiles_m : tile % p.tiles_n) * BN;
  const int64_t M = p.M, N = p.N, K = p.K;
  const int nk_all = (int)(K / kBK);
  const int ks0 = (int)((int64_t)nk_all * split / p.splits);
  const int nk = (int)((int64_t)nk_all * (split + 1) / p.splits) - ks0;

  if (!REDUCE && producer) {
    // =========================== producer waves ===========================
    const int pt = tid - ROLE;
    if (!F16B && pt < 256) {
      pair_lut[pt] = f32x2{p.nf4[pt >> 4], p.nf4[pt & 15]};
      c2t[pt] = p.code2[pt];
    }

    constexpr int B_TOTAL = BN * kBK / BU;                   // W units per tile (a power of 2)
    constexpr int B_UNITS = B_TOTAL / ROLE > 0 ? B_TOTAL / ROLE : 1;  // units per thread
    constexpr int UPR = TRANS ? BN / BU : kBK / BU;   // units per W-tile row
    constexpr int B16 = F16B ? BN * kBK / 8 / ROLE : 1;   // fp16 W chunks (16 bytes) per thread
    struct Stage {
      u32x4 a_reg[A_CHUNKS];
      uint32_t b_word[B_UNITS][BU_WORDS];
      uint32_t b_code[B_UNITS];
      float b_s2[B_UNITS];
      float b_o2[B_UNITS];
      u32x4 b16[B16];
    };
    // fp16 W chunk c of the tile: NT row n (8 chunks of 8 k), NN row k (BN / 8 chunks of 8 n)
    constexpr int B16_PER_ROW = TRANS ? BN / 8 : kBK / 8;
    struct Looked {
      f32x2 v[B_UNITS][BU / 2];
      float c2[B_UNITS];
    };

    // Every load is unconditional (rows past M read row M - 1, whose products land only in
    // output rows that are never stored; steps past the last repeat it), so the compiler counts
    // outstanding loads exactly and waits only for the stage it consumes.
    auto load_tiles = [&](Stage& sg, int kt) {
      const int64_t k0 = (int64_t)(ks0 + (kt < nk ? kt : nk - 1)) * kBK;
#pragma unroll
      for (int i = 0; i < A_CHUNKS; ++i) {
        const int c = pt + ROLE * i;
        const int row = c >> 3, col8 = c & 7;
        const int64_t gm = m0 + row < M ? m0 + row : M - 1;
        sg.a_reg[i] = *reinterpret_cast<const u32x4*>(p.a + gm * p.lda + k0 + col8 * 8);
      }
      if constexpr (F16B) {
#pragma unroll
        for (int i = 0; i < B16; ++i) {
          const int c = pt + ROLE * i;
          const int row = c / B16_PER_ROW, off = (c % B16_PER_ROW) * 8;
          int64_t src;
          if (!TRANS) {
            int64_t n = n0 + row;
            if (EPI == EPI_SWIGLU_FWD) {
              const int64_t g = n >> 6, w = n & 63;
              n = w < 32 ? g * 32 + w : p.inter + g * 32 + (w - 32);
            }
            src = n * K + k0 + off;
          } else {
            src = (k0 + row) * N + n0 + off;
          }
          sg.b16[i] = *reinterpret_cast<const u32x4*>(p.w16 + src);
        }
        return;
      }
#pragma unroll
      for (int i = 0; i < B_UNITS; ++i) {
        // unit c: BU consecutive weights of one stored row, inside one first-level block.
        // NT: row n of W (K contiguous); NN: row k of W (N contiguous).
        const int c = (pt + ROLE * i) & (B_TOTAL - 1);
        const int row = c / UPR, off = (c % UPR) * BU;
        int64_t elem;
        if (!TRANS) {
          int64_t n = n0 + row;
          if (EPI == EPI_SWIGLU_FWD) {
            const int64_t g = n >> 6, w = n & 63;
            n = w < 32 ? g * 32 + w : p.inter + g * 32 + (w - 32);
          }
          elem = n * K + k0 + off;
        } else {
          elem = (k0 + row) * N + n0 + off;
        }
        if constexpr (BU_WORDS == 4) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(p.packed + (elem >> 1));
#pragma unroll
          for (int d = 0; d < 4; ++d) sg.b_word[i][d] = v[d];
        } else {
          const u32x2 v = *reinterpret_cast<const u32x2*>(p.packed + (elem >> 1));
          sg.b_word[i][0] = v[0];
          sg.b_word[i][1] = v[1];
        }
        const int64_t q = elem >> 6;
        sg.b_code[i] = p.qabs[q];
        sg.b_s2[i] = p.scale2[q >> 8];
        sg.b_o2[i] = p.offset2[q >> 8];
      }
    };

    auto look_up = [&](const Stage& sg, Looked& lk) {
      if constexpr (F16B) return;
#pragma unroll
      for (int i = 0; i < B_UNITS; ++i) {
#pragma unroll
        for (int d = 0; d < BU_WORDS; ++d)
#pragma unroll
          for (int bb = 0; bb < 4; ++bb) lk.v[i][4 * d + bb] = pair_lut[(sg.b_word[i][d] >> (8 * bb)) & 0xffu];
        lk.c2[i] = c2t[sg.b_code[i]];
      }
    };

    auto store_tiles = [&](const Stage& sg, const Looked& lk, int buf) {
      f16* as = As[buf];
      f16* bs = Bs[buf];
#pragma unroll
      for (int i = 0; i < A_CHUNKS; ++i) {
        const int c = pt + ROLE * i;
        const int row = c >> 3, col8 = c & 7;
        *reinterpret_cast<u32x4*>(as + row * kStride + col8 * 8) = sg.a_reg[i];
      }
      if constexpr (F16B) {
#pragma unroll
        for (int i = 0; i < B16; ++i) {
          const int c = pt + ROLE * i;
          *reinterpret_cast<u32x4*>(bs + (c / B16_PER_ROW) * B_LD + (c % B16_PER_ROW) * 8) = sg.b16[i];
        }
        return;
      }
#pragma unroll
      for (int i = 0; i < B_UNITS; ++i) {
        // NT: W-tile row n holds k contiguous (the MFMA operand layout); NN: W-tile row k holds
        // n contiguous (the consumers read it with transposing LDS loads)
        const int c = pt + ROLE * i;
        if (c < B_TOTAL) {
          f16* dst = bs + (c / UPR) * B_LD + (c % UPR) * BU;
          const float amax = dk_absmax(lk.c2[i], sg.b_s2[i], sg.b_o2[i]);
#pragma unroll
          for (int d = 0; d < BU_WORDS; ++d) {
            u32x4 o;
#pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
              const f32x2 nv = lk.v[i][4 * d + bb];
              o[bb] = dk_pack2(dk_h(__fmul_rn(nv[0], amax)), dk_h(__fmul_rn(nv[1], amax)));
            }
            *reinterpret_cast<u32x4*>(dst + d * 8) = o;
          }
        }
      }
    };

    // Step j lives in register stage j % 3 and LDS buffer j % 2.  While the consumers run step
    // j, the producers issue the loads of step j + 3 into the stage step j has vacated and write
    // step j + 1 into the other buffer; each load has two steps of MFMA time to land.  Steps past
    // the last repeat it into a buffer that is not read again: no branch around memory
    // operations inside the loop.
    if constexpr (F16B) {
      // fp16 W: 32 registers per stage, so two stages.  Step j + 1 is in one stage while step
      // j + 2 loads into the other; each load has one step of MFMA time to land.
      Stage s0, s1;
      Looked lk;
      load_tiles(s0, 0);
      load_tiles(s1, 1);
      __syncthreads();
      store_tiles(s0, lk, 0);
      __syncthreads();  // step 0 in buffer 0
      int j = 0;
      for (; j + 2 <= nk; j += 2) {
        load_tiles(s0, j + 2);
        store_tiles(s1, lk, (j + 1) & 1);
        __syncthreads();
        load_tiles(s1, j + 3);
        store_tiles(s0, lk, j & 1);
        __syncthreads();
      }
      if (j < nk) {
        store_tiles(s1, lk, (j + 1) & 1);
        __syncthreads();
      }
      return;
    }
    Stage s0, s1, s2;
    Looked lk;
    load_tiles(s0, 0);
    load_tiles(s1, 1);
    load_tiles(s2, 2);
    __syncthreads();  // lookup tables visible
    look_up(s0, lk);
    store_tiles(s0, lk, 0);
    __syncthreads();  // step 0 in buffer 0
    int j = 0;
    for (; j + 3 <= nk; j += 3) {
      load_tiles(s0, j + 3);
      look_up(s1, lk);
      store_tiles(s1, lk, (j + 1) & 1);
      __syncthreads();
      load_tiles(s1, j + 4);
      look_up(s2, lk);
      store_tiles(s2, lk, j & 1);
      __syncthreads();
      load_tiles(s2, j + 5);
      look_up(s0, lk);
      store_tiles(s0, lk, (j + 1) & 1);
      __syncthreads();
    }
    if (j < nk) {
      look_up(s1, lk);
      store_tiles(s1, lk, (j + 1) & 1);
      __syncthreads();
    }
    if (j + 1 < nk) {
      look_up(s2, lk);
      store_tiles(s2, lk, j & 1);
      __syncthreads();
    }
    return;
  }

  // =========================== consumer waves ===========================
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int lrow = lane & 31;
  const int lk8 = 8 * (lane >> 5);
  const int rsub = 4 * (lane >> 5);
  // NN transposing reads: this lane's row and column offsets in the W tile (see compute)
  const int tr_k = 8 * (lane >> 5) + ((lane & 15) >> 2);
  const int tr_n = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  // ---- epilogue of one 32 x 32 block (i, j) of this wave's sub-tile.  Lane layout of a 32 x 32
  // fp32 MFMA result: column lane % 32, row 8 * (v / 4) + 4 * (lane / 32) + v % 4 for register v.
  // this consumer wave's 4 KB of epilogue scratch in LDS (keep-mask bytes at 0, a LoRA A slice
  // at 2048): after the last K-step the A tile buffers are free (every producer store and
  // consumer read is behind the final barrier)
  constexpr int kEpiScratch = 4096;
  static_assert(WAVES_M * WAVES_N * kEpiScratch <= BM * kStride * 2, "epilogue scratch");
  uint8_t* escr;
  if constexpr (REDUCE) {
    __shared__ __attribute__((aligned(16))) uint8_t reduce_scr[WAVES_M * WAVES_N][kEpiScratch];
    escr = reduce_scr[wave];
  } else {
    escr = reinterpret_cast<uint8_t*>(As[0]) + wave * kEpiScratch;
  }

  auto linear_block = [&](int i, int j, const f32x16& a) {
    f16* out16 = reinterpret_cast<f16*>(p.out);
    float* out32 = reinterpret_cast<float*>(p.out);
    const int64_t mrow0 = m0 + wm * WM + 32 * i;
    const int64_t nb = n0 + wn * WN + 32 * j;  // first column of the block
    const int64_t n = nb + lrow;
    const float bias = p.bias ? (float)p.bias[n] : 0.0f;
    f32x16 res;
#pragma unroll
    for (int v = 0; v < 16; ++v) res[v] = (float)dk_h(__fadd_rn(a[v], bias));
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (t >= p.n_lora) break;
      const LoraTerm& L = p.lora[t];
      if (!TRANS && (nb < L.n_begin || nb >= L.n_end)) continue;
      f32x16 lo;
#pragma unroll
      for (int v = 0; v < 16; ++v) lo[v] = 0.0f;
      const int64_t zm = mrow0 + lrow;
      for (int rc = 0; rc < p.rank; rc += 16) {
        f16x8 zf, rf;
        if (zm < M) {
          zf = *reinterpret_cast<const f16x8*>(L.z + zm * p.rank + rc + lk8);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) zf[e] = (f16)0.0f;
        }
        if (!TRANS) {
          rf = *reinterpret_cast<const f16x8*>(L.r + (n - L.n_begin) * p.rank + rc + lk8);
        } else {
          // A[rc .. rc + 16][nb .. nb + 32] staged row-major in LDS (one 16-byte load per lane,
          // rows of 48 halves) and read back rank-contiguous with transposing reads, as the W
          // tile of the main loop
          f16* ascr = reinterpret_cast<f16*>(escr + 2048);
          const f16x8 av = *reinterpret_cast<const f16x8*>(
              L.r + (int64_t)(rc + (lane >> 2)) * N + nb + 8 * (lane & 3));
          __builtin_amdgcn_wave_barrier();
          *reinterpret_cast<f16x8*>(ascr + (lane >> 2) * 48 + 8 * (lane & 3)) = av;
          __builtin_amdgcn_wave_barrier();
          const f16* base = ascr + tr_k * 48 + tr_n;
          const f16x4 lo4 = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(base)));
          const f16x4 hi4 = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(base + 4 * 48)));
          rf = f16x8{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
          __builtin_amdgcn_wave_barrier();
        }
        lo = __builtin_amdgcn_mfma_f32_32x32x16_f16(zf, rf, lo, 0, 0, 0);
      }
      if (TRANS && L.mask) {
        // the block's 32 x 32 keep-mask bytes: one coalesced 16-byte load per lane, staged in
        // this wave's LDS scratch (rows of 48 bytes), then read per element
        const int64_t mr = mrow0 + (lane >> 1);
        u32x4 mw = u32x4{0u, 0u, 0u, 0u};
        if (mr < M) mw = *reinterpret_cast<const u32x4*>(L.mask + mr * N + nb + 16 * (lane & 1));
        __builtin_amdgcn_wave_barrier();
        *reinterpret_cast<u32x4*>(escr + (lane >> 1) * 48 + 16 * (lane & 1)) = mw;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int mloc = 8 * (v >> 2) + rsub + (v & 3);
          const float lf = (float)dk_h(lo[v]);
          res[v] = __fadd_rn(res[v], escr[mloc * 48 + lrow] ? __fmul_rn(lf, L.scale) : 0.0f);
        }
        __builtin_amdgcn_wave_barrier();
      } else {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float lf = (float)dk_h(lo[v]);
          res[v] = __fadd_rn(res[v], TRANS ? lf : __fmul_rn(L.scale, lf));
        }
      }
    }
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int64_t m = mrow0 + 8 * (v >> 2) + rsub + (v & 3);
      if (m >= M) continue;
      const int64_t o = m * p.ldo + n;
      if (p.out_mode == DK_OUT_F16) {
        out16[o] = dk_h(res[v]);
      } else if (p.out_mode == DK_OUT_F32) {
        out32[o] = res[v];
      } else {
        out32[o] = __fadd_rn(out32[o], res[v]);
      }
    }
  };

  if constexpr (REDUCE) {
    // split-K, second launch: block (i, j) of every consumer sub-tile of the tile, the partials
    // summed in split order (a fixed order, so the result is deterministic); the kernel boundary
    // orders this launch after every partial store
    static_assert(EPI == EPI_LINEAR, "split-K runs the linear epilogue only");
    const int ij = b % per_tile;
    const int i = ij / TN, j = ij % TN;
    const float* all = p.part + (int64_t)tile * p.splits * TILE +
                       ((wave * TM + i) * TN + j) * 16 * 64 + lane;
    f32x16 a;
#pragma unroll
    for (int v = 0; v < 16; ++v) a[v] = all[v * 64];
    for (int sp = 1; sp < p.splits; ++sp) {
#pragma unroll
      for (int v = 0; v < 16; ++v) a[v] += all[(int64_t)sp * TILE + v * 64];
    }
    linear_block(i, j, a);
    return;
  } else {
    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    struct Frags {
      f16x8 a[TM], b[TN];
    };
    // the MFMA operands of K sub-step s (16 wide) of LDS buffer buf
    auto load_frags = [&](Frags& f, int buf, int s) {
      const f16* as = As[buf];
      const f16* bs = Bs[buf];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        f.a[i] = *reinterpret_cast<const f16x8*>(as + (wm * WM + 32 * i + lrow) * kStride + 16 * s + lk8);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if (!TRANS) {
          f.b[j] = *reinterpret_cast<const f16x8*>(bs + (wn * WN + 32 * j + lrow) * kStride + 16 * s + lk8);
        } else {
          // ds_read_b64_tr_b16: within each 16-lane group, lane 4a + b receives element b of the
          // 4-element rows addressed by lanes a, a + 4, a + 8, a + 12.  Lane 4j + a of group G
          // addresses row k = 16 s + 8 (G / 2) + 4 h + j, columns from 16 (G % 2) + 4 a, so lane
          // l gets W[k0 + 8 (l / 32) + 4 h + 0..3][l % 32]: two reads (h = 0, 1) give the 8
          // consecutive k of the MFMA operand.
          const f16* base = bs + (16 * s + tr_k) * B_LD + wn * WN + 32 * j + tr_n;
          const f16x4 lo = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(base)));
          const f16x4 hi = __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (__attribute__((address_space(3))) i16x4*)(base + 4 * B_LD)));
          f.b[j] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
    };
    auto mma = [&](const Frags& f) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f.a[i], f.b[j], acc[i][j], 0, 0, 0);
    };
    // The same number of barriers as the producers: 2 before step 0, one per step.  Software
    // pipelined by one K sub-step: the operands of sub-step s + 1 are read while the MFMAs of s
    // run.  The step's last operands are in registers at its barrier (which waits for every LDS
    // read), so its last MFMAs run after the barrier, beside the first reads of the next step.
    __syncthreads();
    __syncthreads();
    Frags f0, f1;
    load_frags(f0, 0, 0);
    for (int kt = 0; kt < nk; ++kt) {
      const int buf = kt & 1;
      load_frags(f1, buf, 1);
      mma(f0);
      load_frags(f0, buf, 2);
      mma(f1);
      load_frags(f1, buf, 3);
      mma(f0);
      __syncthreads();
      if (kt + 1 < nk) load_frags(f0, buf ^ 1, 0);
      mma(f1);
    }

    // split-K, first launch: store the fp32 partial tile (lane-major, so each register store is
    // 256 contiguous bytes) and stop; the epilogue runs in the second launch
    if (p.splits > 1) {
      float* mine = p.part + ((int64_t)tile * p.splits + split) * TILE;
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            mine[(((wave * TM + i) * TN + j) * 16 + v) * 64 + lane] = acc[i][j][v];
      return;
    }

    if constexpr (EPI == EPI_LINEAR) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) linear_block(i, j, acc[i][j]);
    } else if constexpr (EPI == EPI_SWIGLU_FWD) {
      f16* act = reinterpret_cast<f16*>(p.out);
      const int64_t hcol = (n0 + wn * WN) / 2 + lrow;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int64_t mrow0 = m0 + wm * WM + 32 * i;
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int64_t m = mrow0 + 8 * (v >> 2) + rsub + (v & 3);
          if (m >= M) continue;
          const f16 g16 = dk_h(acc[i][0][v]);
          const f16 u16 = dk_h(acc[i][1][v]);
          float sig, silu;
          dk_silu_parts((float)g16, &sig, &silu);
          act[m * p.ldo + hcol] = dk_h(silu * (float)u16);
          if (p.gu) {
            p.gu[m * 2 * p.inter + hcol] = g16;
            p.gu[m * 2 * p.inter + p.inter + hcol] = u16;
          }
        }
      }
    } else {  // EPI_SWIGLU_BWD: N == inter
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int64_t mrow0 = m0 + wm * WM + 32 * i;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int64_t n = n0 + wn * WN + 32 * j + lrow;
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int64_t m = mrow0 + 8 * (v >> 2) + rsub + (v & 3);
            if (m >= M) continue;
            const float da = (float)dk_h(acc[i][j][v]);
            f16* gp = p.gu + m * 2 * p.inter + n;
            const float g = (float)gp[0];
            const float u = (float)gp[p.inter];
            float sig, silu;
            dk_silu_parts(g, &sig, &silu);
            gp[p.inter] = dk_h(da * silu);
            gp[0] = dk_h((da * u) * sig * (1.0f + g * (1.0f - sig)));
          }
        }
      }
    }
  }
}

// Launch plan: tile shape and split-K factor.  256 CUs.  A 128-row tile's workgroup needs
// 76.8 KB of LDS (60 KB at 64 columns) and at most 128 VGPRs, so two share a CU (512 slots).
// (256 x 128 tiles, one workgroup per CU, measured slower at these shapes and are not
// planned.)  Shapes with fewer tiles than slots split K (at least 8 steps per split) so that about
// 768 workgroups run: the fp32 partial tiles cost one extra pass over the output in the second
// launch, so short K (under 64 steps) prefers narrower tiles and splits only below 256 tiles.
struct Plan {
  int bm, bn, splits;
  int64_t tiles;
};

Plan plan_for(int64_t M, int64_t N, int64_t K, int epi) {
  const int64_t nk = K / kBK;
  const int64_t mt128 = (M + 127) / 128;
  Plan pl{128, 128, 1, mt128 * (N / 128)};
  if (N % 128 != 0) pl = {128, 64, 1, mt128 * (N / 64)};
  if (epi != EPI_LINEAR || pl.tiles >= 512) return pl;
  if (pl.bn == 128 && nk < 64) pl = {128, 64, 1, mt128 * (N / 64)};
  if ((pl.tiles < 256 && nk >= 16) || (pl.tiles < 512 && nk >= 64)) {
    int64_t s = (768 + pl.tiles - 1) / pl.tiles;
    if (s > nk / 8) s = nk / 8;
    if (s > 8) s = 8;
    if (s >= 2) pl.splits = (int)s;
  }
  return pl;
}

// Two-phase path: with many row tiles, dequantising each W tile once per row tile (in LDS) costs
// more LDS bandwidth than the MFMAs can hide, so from kTwoPhaseRows rows and kTwoPhaseCols
// output columns on, the weight is first dequantised once into the workspace at HBM rate
// (nf4_dequant_kernel) and the GEMM reads fp16 W (on the 256-tile kernel where it takes the
// shape).  Measured on MI355X at M = 2048 against this file's kernel: gate|up forward
// (N = 17920) 174 -> 153 us, down backward (N = 8960) 139 -> 132 us, and, with the 256-tile
// kernel's 128 x 128 quarters, q|k|v forward 33.3 -> 27.9 us, o forward 30.3 -> 24.7, o dX
// 31.5 -> 24.5, q|k|v dX 42.3 -> 33.4.
constexpr int64_t kTwoPhaseRows = 512;
constexpr int64_t kTwoPhaseCols = 1536;

bool two_phase(int64_t M, int64_t N) { return M >= kTwoPhaseRows && N >= kTwoPhaseCols; }

int64_t round256(int64_t b) { return (b + 255) / 256 * 256; }

int64_t plan_workspace(const Plan& pl) {
  if (pl.splits <= 1) return 0;
  return pl.tiles * pl.splits * pl.bm * pl.bn * (int64_t)sizeof(float);
}

// Workspace of one GEMM: [split-K partial tiles | fp16 weight (two-phase)].
// Workspace of an NF4-reading GEMM: room for whichever path dispatch takes, the 256-tile kernel's
// split-K partials (reading NF4 itself), or the 128 x 128 kernel's partials with the fp16 weight
// after them (two-phase shapes).
int64_t gemm_workspace(int64_t M, int64_t N, int64_t K, int epi, bool nt) {
  if (M <= 0) return 0;
  const int64_t part = plan_workspace(plan_for(M, N, K, epi));
  const int64_t w16 = two_phase(M, N) ? N * K * (int64_t)sizeof(f16) : 0;
  const int64_t own = w16 ? round256(part) + w16 : part;
  const int64_t tile = hgemm_workspace(M, N, K, epi, nt);
  return own > tile ? own : tile;
}

template <int BM, int BN, bool TRANS, int EPI, bool F16B>
int launch(GemmParams p, int splits, hipStream_t stream) {
  p.tiles_n = (int)(p.N / BN);
  p.tiles_m = (int)((p.M + BM - 1) / BM);
  // fp16 W (two-phase) is 4x the bytes of packed W: with row tiles fastest, each XCD's run of
  // tiles covers a band of columns for every row tile, so each XCD reads its slice of W once
  p.m_fastest = F16B ? 1 : 0;
  const int64_t tiles = (int64_t)p.tiles_m * p.tiles_n;
  p.splits = splits;
  constexpr int blocks = 2 * (BN / 64);   // 32 x 32 blocks per consumer sub-tile (64 x BN/2)
  if (tiles <= 0 || tiles * (splits > blocks ? splits : blocks) > 0x7fffffff) return DK_ERR_INVALID;
  if (splits > 1 && EPI != EPI_LINEAR) return DK_ERR_INVALID;
  hipLaunchKernelGGL((w4_gemm_kernel<BM, BN, TRANS, EPI, false, F16B>),
                     dim3((unsigned)(tiles * splits)), dim3(2 * role_threads<BM>()), 0, stream, p);
  DK_CHECK_LAUNCH();
  if constexpr (EPI == EPI_LINEAR) {
    if (splits > 1) {
      hipLaunchKernelGGL((w4_gemm_kernel<BM, BN, TRANS, EPI, true, false>),
                         dim3((unsigned)(tiles * blocks)), dim3(role_threads<BM>()), 0, stream, p);
      DK_CHECK_LAUNCH();
    }
  }
  return 0;
}

template <bool TRANS, int EPI, bool F16B>
int launch_plan(const Plan& pl, GemmParams p, hipStream_t stream) {
  if (pl.bm == 256) return launch<256, 128, TRANS, EPI, F16B>(p, pl.splits, stream);
  if (pl.bn == 128) return launch<128, 128, TRANS, EPI, F16B>(p, pl.splits, stream);
  if constexpr (EPI == EPI_SWIGLU_FWD) {
    return DK_ERR_INVALID;
  } else {
    return launch<128, 64, TRANS, EPI, F16B>(p, pl.splits, stream);
  }
}

// Runs the plan.  Without a workspace: one phase (W dequantised in LDS), no split-K.  With one
// (at least gemm_workspace bytes): split-K partials and, on the two-phase shapes, the weight
// dequantised to fp16 in the workspace first (both launches on `stream`, in order).  The weight's
// `kernel` field picks the 256-tile kernel reading NF4: where it is fastest (AUTO: split-K
// plans), wherever its plan takes the shape (TILE), or never (STAGED).

template <bool TRANS, int EPI>
int dispatch(GemmParams p, const dk_nf4_weight* w, void* ws, int64_t ws_bytes, hipStream_t stream) {
  if (ws && ws_bytes < gemm_workspace(p.M, p.N, p.K, EPI, !TRANS)) return DK_ERR_WORKSPACE;
  // the 256-tile kernel with the weight dequantised in LDS (W4) where its plan splits K (few
  // output tiles, long K): there it beats the separate dequant + fp16 GEMM (gate|up dX at
  // M = 2048: 179 against 188 us); elsewhere its per-step conversion costs more than the
  // dequant launch saves (measured on every config-4 shape), and the paths below run
  const int mode = w->kernel;
  if (mode == DK_W4_KERNEL_TILE ||
      (mode == DK_W4_KERNEL_AUTO && ws && hgemm_workspace(p.M, p.N, p.K, EPI, !TRANS) > 0)) {
    const int r = hgemm_launch<TRANS, EPI, true>(p, ws, ws_bytes, stream);
    if (r != kHgemmDeclined) return r;
  }
  Plan pl = plan_for(p.M, p.N, p.K, EPI);
  if (ws == nullptr) {
    pl.splits = 1;
    return launch_plan<TRANS, EPI, false>(pl, p, stream);
  }
  if (ws_bytes < gemm_workspace(p.M, p.N, p.K, EPI, !TRANS)) return DK_ERR_WORKSPACE;
  if (!dk_aligned(ws, 256)) return DK_ERR_ALIGN;
  if (pl.splits > 1) p.part = reinterpret_cast<float*>(ws);
  if (!two_phase(p.M, p.N)) return launch_plan<TRANS, EPI, false>(pl, p, stream);
  f16* w16 = reinterpret_cast<f16*>(reinterpret_cast<char*>(ws) + round256(plan_workspace(pl)));
  if (int e = dk_nf4_dequant(w->packed, w->qabs, w->scale2, w->offset2, w->code2, w->nf4, w16,
                             w->rows * w->cols / DK_QBLOCK, stream))
    return e;
  p.w16 = w16;
  const int big = hgemm_launch<TRANS, EPI>(p, nullptr, 0, stream);
  if (big != kHgemmDeclined) return big;
  return launch_plan<TRANS, EPI, true>(pl, p, stream);
}

bool weight_ok(const dk_nf4_weight* w) {
  return w && w->packed && w->qabs && w->scale2 && w->offset2 && w->code2 && w->nf4 &&
         w->rows > 0 && w->cols > 0 && (w->rows * w->cols) % DK_ELEMS_PER_SB == 0 &&
         w->kernel >= DK_W4_KERNEL_AUTO && w->kernel <= DK_W4_KERNEL_STAGED;
}

void set_weight(GemmParams& p, const dk_nf4_weight* w) {
  p.packed = w->packed;
  p.qabs = w->qabs;
  p.scale2 = w->scale2;
  p.offset2 = w->offset2;
  p.code2 = w->code2;
  p.nf4 = w->nf4;
}

// Copies the caller's LoRA terms into the kernel parameters.  Forward terms cover disjoint
// column ranges, multiples of 32 inside [0, n_cols); backward terms cover every column.
int set_lora(GemmParams& p, const dk_lora_term* terms, int n_terms, int64_t rank, int64_t n_cols,
             bool backward) {
  if (n_terms < 0 || n_terms > 2 || (n_terms > 0 && !terms)) return DK_ERR_INVALID;
  if (n_terms > 0 && (rank < 16 || rank > 64 || rank % 16)) return DK_ERR_INVALID;
  p.n_lora = n_terms;
  p.rank = rank;
  for (int t = 0; t < n_terms; ++t) {
    const dk_lora_term& u = terms[t];
    if (!u.left || !u.right) return DK_ERR_INVALID;
    if (!dk_aligned(u.left, 16) || !dk_aligned(u.right, 16)) return DK_ERR_ALIGN;
    if (backward && u.mask && !dk_aligned(u.mask, 16)) return DK_ERR_ALIGN;
    LoraTerm& L = p.lora[t];
    L.z = (const f16*)u.left;
    L.r = (const f16*)u.right;
    if (backward) {
      L.mask = u.mask;
      L.scale = u.mask ? u.scale : 1.0f;
      L.n_begin = 0;
      L.n_end = n_cols;
    } else {
      if (u.mask) return DK_ERR_INVALID;
      if (u.col_begin < 0 || u.col_end > n_cols || u.col_begin >= u.col_end ||
          u.col_begin % 32 || u.col_end % 32)
        return DK_ERR_INVALID;
      for (int q = 0; q < t; ++q)
        if (u.col_begin < p.lora[q].n_end && p.lora[q].n_begin < u.col_end) return DK_ERR_INVALID;
      L.mask = nullptr;
      L.scale = u.scale;
      L.n_begin = u.col_begin;
      L.n_end = u.col_end;
    }
  }
  return 0;
}


// ---- parameter set-up shared by the NF4 (dk_w4_*) and fp16 (dk_h16_*) entry points; rows x
// cols is the stored weight shape [out, in].

int linear_fwd_params(GemmParams& p, const void* x, int64_t ldx, int64_t m, int64_t rows,
                      int64_t cols, const void* bias, const dk_lora_term* terms, int n_terms,
                      int64_t rank, void* y, int64_t ldy) {
  if (m < 0 || !x || !y || rows <= 0 || cols <= 0) return DK_ERR_INVALID;
  if (rows % 64 || cols % kBK || ldx < cols || ldy < rows) return DK_ERR_INVALID;
  if (!dk_aligned(x, 16) || ldx % 8) return DK_ERR_ALIGN;
  if (int e = set_lora(p, terms, n_terms, rank, rows, false)) return e;
  p.a = (const f16*)x;
  p.lda = ldx;
  p.M = m;
  p.N = rows;
  p.K = cols;
  p.bias = (const f16*)bias;
  p.out = y;
  p.ldo = ldy;
  p.out_mode = DK_OUT_F16;
  return 0;
}

int linear_bwd_params(GemmParams& p, const void* dy, int64_t lddy, int64_t m, int64_t rows,
                      int64_t cols, const dk_lora_term* terms, int n_terms, int64_t rank,
                      void* dx, int64_t lddx, int out_mode) {
  if (m < 0 || !dy || !dx || rows <= 0 || cols <= 0) return DK_ERR_INVALID;
  if (out_mode < DK_OUT_F16 || out_mode > DK_OUT_F32_ACCUM) return DK_ERR_INVALID;
  if (cols % 64 || rows % kBK || lddy < rows || lddx < cols) return DK_ERR_INVALID;
  if (!dk_aligned(dy, 16) || lddy % 8) return DK_ERR_ALIGN;
  if (int e = set_lora(p, terms, n_terms, rank, cols, true)) return e;
  p.a = (const f16*)dy;
  p.lda = lddy;
  p.M = m;
  p.N = cols;
  p.K = rows;
  p.out = dx;
  p.ldo = lddx;
  p.out_mode = out_mode;
  return 0;
}

int gateup_params(GemmParams& p, const void* x, int64_t ldx, int64_t m, int64_t rows,
                  int64_t cols, void* act, void* gu_out) {
  if (m < 0 || !x || !act || rows <= 0 || cols <= 0) return DK_ERR_INVALID;
  if (rows % 128 || cols % kBK || ldx < cols) return DK_ERR_INVALID;
  if (!dk_aligned(x, 16) || ldx % 8) return DK_ERR_ALIGN;
  p.a = (const f16*)x;
  p.lda = ldx;
  p.M = m;
  p.N = rows;  // logical columns: 2 * inter, interleaved in groups of 32
  p.K = cols;
  p.inter = rows / 2;
  p.out = act;
  p.ldo = p.inter;
  p.gu = (f16*)gu_out;
  return 0;
}

int down_bwd_params(GemmParams& p, const void* dh, int64_t lddh, int64_t m, int64_t rows,
                    int64_t cols, void* gu) {
  if (m < 0 || !dh || !gu || rows <= 0 || cols <= 0) return DK_ERR_INVALID;
  if (cols % 64 || rows % kBK || lddh < rows) return DK_ERR_INVALID;
  if (!dk_aligned(dh, 16) || lddh % 8) return DK_ERR_ALIGN;
  p.a = (const f16*)dh;
  p.lda = lddh;
  p.M = m;
  p.N = cols;  // inter
  p.K = rows;  // d_model
  p.inter = cols;
  p.gu = (f16*)gu;
  return 0;
}

// Checks the dequant work a launch carries and copies it into the kernel parameters.
int set_side(GemmParams& p, const dk_side_dequant* side) {
  p.side = SideDequant{};
  if (!side || side->wgs == 0 || side->sb0 == side->sb1) return 0;
  if ((side->wgs < 1 && side->wgs != DK_SIDE_WGS_AUTO) || side->wgs > 1024 || side->sb0 < 0 ||
      side->sb1 < side->sb0)
    return DK_ERR_INVALID;
  if (!side->packed || !side->qabs || !side->scale2 || !side->offset2 || !side->code2 ||
      !side->nf4 || !side->out)
    return DK_ERR_INVALID;
  if (!dk_aligned(side->packed, 16) || !dk_aligned(side->out, 16)) return DK_ERR_ALIGN;
  p.side.packed = reinterpret_cast<const u32x4*>(side->packed);
  p.side.qabs = side->qabs;
  p.side.scale2 = side->scale2;
  p.side.offset2 = side->offset2;
  p.side.code2 = side->code2;
  p.side.nf4 = side->nf4;
  p.side.out = reinterpret_cast<u32x4*>(side->out);
  p.side.sb0 = side->sb0;
  p.side.sb1 = side->sb1;
  p.side.wgs = side->wgs;
  return 0;
}

// The carried dequant as a launch of its own, for GEMMs that do not run on the 256 x 256-tile
// kernel (the same blocks, bit for bit).
int side_alone(const SideDequant& s, hipStream_t stream) {
  if (s.wgs == 0) return 0;
  const int64_t q0 = s.sb0 * DK_QBLOCK2;
  return dk_nf4_dequant(reinterpret_cast<const uint8_t*>(s.packed) + q0 * 32, s.qabs + q0,
                        s.scale2 + s.sb0, s.offset2 + s.sb0, s.code2, s.nf4,
                        reinterpret_cast<f16*>(s.out) + q0 * DK_QBLOCK, (s.sb1 - s.sb0) * DK_QBLOCK2,
                        stream);
}

// fp16 weight: the 256 x 256-tile kernel where the shape suits it (no workspace), else the plan's
// split-K (partials in the workspace when one is given), one phase.
// LoRA column sums a dX GEMM carries (dk_side_lora_sums), or none; blocks: their workgroups.
struct CarriedSums {
  SumJobs jobs;
  int blocks = 0;
  int64_t rows = 0, rank = 0;
};

int set_sums(CarriedSums& c, const dk_side_lora_sums* sums) {
  if (!sums) return 0;
  c.rows = sums->m;
  c.rank = sums->rank;
  return lora_sum_jobs(sums->x, sums->m, sums->k, sums->rank, sums->terms, sums->n_terms, &c.jobs,
                       &c.blocks);
}

// fp16 weight: the 256 x 256-tile kernel where the shape suits it (no workspace), else the plan's
// split-K (partials in the workspace when one is given), one phase.  Carried work (side dequant,
// LoRA column sums) joins the 256-tile launch, or runs after the GEMM in launches of its own.
template <bool TRANS, int EPI>
int dispatch_h16(GemmParams p, const void* w16, void* ws, int64_t ws_bytes,
                 const dk_side_dequant* side, hipStream_t stream,
                 const CarriedSums& sums = CarriedSums{}) {
  if (!w16) return DK_ERR_INVALID;
  if (!dk_aligned(w16, 16)) return DK_ERR_ALIGN;
  if (int e = set_side(p, side)) return e;
  auto sums_alone = [&]() {
    return sums.blocks ? lora_sums_launch(sums.rank, sums.jobs, sums.blocks, sums.rows, stream) : 0;
  };
  if (p.M == 0) {
    if (int e = side_alone(p.side, stream)) return e;
    return sums_alone();
  }
  p.w16 = (const f16*)w16;
  // the 256-tile kernel carries rank-16 column sums of NN LINEAR GEMMs
  const bool carry = sums.blocks > 0 && sums.rank == 16 && TRANS && EPI == EPI_LINEAR;
  if (carry) {
    p.sums.jobs = sums.jobs;
    p.sums.rows = sums.rows;
    p.sums.wgs = sums.blocks;
  }
  const int big = hgemm_launch<TRANS, EPI>(p, ws, ws_bytes, stream);
  if (big != kHgemmDeclined) return big ? big : (carry ? 0 : sums_alone());
  p.sums = SideSums{};
  Plan pl = plan_for(p.M, p.N, p.K, EPI);
  if (ws == nullptr) {
    pl.splits = 1;
  } else if (pl.splits > 1) {
    if (ws_bytes < plan_workspace(pl)) return DK_ERR_WORKSPACE;
    if (!dk_aligned(ws, 256)) return DK_ERR_ALIGN;
    p.part = reinterpret_cast<float*>(ws);
  }
  if (int e = launch_plan<TRANS, EPI, true>(pl, p, stream)) return e;
  if (int e = side_alone(p.side, stream)) return e;
  return sums_alone();
}

template <bool TRANS, int EPI>
int dispatch_w4(GemmParams p, const dk_nf4_weight* w, void* ws, int64_t ws_bytes,
                hipStream_t stream) {
  if (!weight_ok(w)) return DK_ERR_INVALID;
  if (!dk_aligned(w->packed, 16)) return DK_ERR_ALIGN;
  if (p.M == 0) return 0;
  set_weight(p, w);
  return dispatch<TRANS, EPI>(p, w, ws, ws_bytes, stream);
}

}  // namespace

extern "C" int dk_w4_linear_fwd_lora(const void* x, int64_t ldx, int64_t m,
                                     const dk_nf4_weight* w, const void* bias,
                                     const dk_lora_term* terms, int n_terms, int64_t rank,
                                     void* y, int64_t ldy, void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream) {
  if (!weight_ok(w)) return DK_ERR_INVALID;
  GemmParams p = {};
  if (int e = linear_fwd_params(p, x, ldx, m, w->rows, w->cols, bias, terms, n_terms, rank, y, ldy))
    return e;
  return dispatch_w4<false, EPI_LINEAR>(p, w, workspace, workspace_bytes, stream);
}

extern "C" int dk_w4_linear_fwd(const void* x, int64_t ldx, int64_t m, const dk_nf4_weight* w,
                                const void* bias, const void* z, const void* lora_b,
                                int64_t rank, float lora_scale, void* y, int64_t ldy,
                                void* workspace, int64_t workspace_bytes, hipStream_t stream) {
  if ((z == nullptr) != (lora_b == nullptr) || !weight_ok(w)) return DK_ERR_INVALID;
  dk_lora_term t = {z, lora_b, nullptr, 0, w->rows, lora_scale};
  return dk_w4_linear_fwd_lora(x, ldx, m, w, bias, &t, z ? 1 : 0, z ? rank : 0, y, ldy,
                               workspace, workspace_bytes, stream);
}

extern "C" int dk_w4_linear_bwd_dx_lora(const void* dy, int64_t lddy, int64_t m,
                                        const dk_nf4_weight* w, const dk_lora_term* terms,
                                        int n_terms, int64_t rank, void* dx, int64_t lddx,
                                        int out_mode, void* workspace, int64_t workspace_bytes,
                                        hipStream_t stream) {
  if (!weight_ok(w)) return DK_ERR_INVALID;
  GemmParams p = {};
  if (int e = linear_bwd_params(p, dy, lddy, m, w->rows, w->cols, terms, n_terms, rank, dx, lddx,
                                out_mode))
    return e;
  return dispatch_w4<true, EPI_LINEAR>(p, w, workspace, workspace_bytes, stream);
}

extern "C" int dk_w4_linear_bwd_dx(const void* dy, int64_t lddy, int64_t m,
                                   const dk_nf4_weight* w, const void* dz, const void* lora_a,
                                   int64_t rank, const uint8_t* mask, float keep_scale, void* dx,
                                   int64_t lddx, int out_mode, void* workspace,
                                   int64_t workspace_bytes, hipStream_t stream) {
  if ((dz == nullptr) != (lora_a == nullptr)) return DK_ERR_INVALID;
  dk_lora_term t = {dz, lora_a, mask, 0, 0, keep_scale};
  return dk_w4_linear_bwd_dx_lora(dy, lddy, m, w, &t, dz ? 1 : 0, dz ? rank : 0, dx, lddx,
                                  out_mode, workspace, workspace_bytes, stream);
}

extern "C" int dk_w4_gateup_swiglu_fwd(const void* x, int64_t ldx, int64_t m,
                                       const dk_nf4_weight* w_gu, void* act, void* gu_out,
                                       void* workspace, int64_t workspace_bytes,
                                       hipStream_t stream) {
  if (!weight_ok(w_gu)) return DK_ERR_INVALID;
  GemmParams p = {};
  if (int e = gateup_params(p, x, ldx, m, w_gu->rows, w_gu->cols, act, gu_out)) return e;
  return dispatch_w4<false, EPI_SWIGLU_FWD>(p, w_gu, workspace, workspace_bytes, stream);
}

extern "C" int dk_w4_down_swiglu_bwd(const void* dh, int64_t lddh, int64_t m,
                                     const dk_nf4_weight* w_down, void* gu, void* workspace,
                                     int64_t workspace_bytes, hipStream_t stream) {
  if (!weight_ok(w_down)) return DK_ERR_INVALID;
  GemmParams p = {};
  if (int e = down_bwd_params(p, dh, lddh, m, w_down->rows, w_down->cols, gu)) return e;
  return dispatch_w4<true, EPI_SWIGLU_BWD>(p, w_down, workspace, workspace_bytes, stream);
}

// ---- fp16 weights (the reference's GEMMs on its dequantised workspace)

extern "C" int dk_h16_linear_fwd_lora(const void* x, int64_t ldx, int64_t m, const void* w16,
                                      int64_t rows, int64_t cols, const void* bias,
                                      const dk_lora_term* terms, int n_terms, int64_t rank,
                                      void* y, int64_t ldy, void* workspace,
                                      int64_t workspace_bytes, const dk_side_dequant* side,
                                      hipStream_t stream) {
  GemmParams p = {};
  if (int e = linear_fwd_params(p, x, ldx, m, rows, cols, bias, terms, n_terms, rank, y, ldy))
    return e;
  return dispatch_h16<false, EPI_LINEAR>(p, w16, workspace, workspace_bytes, side, stream);
}

extern "C" int dk_h16_linear_fwd_rope(const void* x, int64_t ldx, int64_t m, const void* w16,
                                      int64_t rows, int64_t cols, const void* bias,
                                      const dk_lora_term* terms, int n_terms, int64_t rank,
                                      const dk_rope* rope, void* y, int64_t ldy,
                                      const dk_side_dequant* side, hipStream_t stream) {
  GemmParams p = {};
  if (int e = linear_fwd_params(p, x, ldx, m, rows, cols, bias, terms, n_terms, rank, y, ldy))
    return e;
  if (!rope || !rope->pos || !rope->cos_table || !rope->sin_table || !w16) return DK_ERR_INVALID;
  if (rope->hd != 128 || rope->cols <= 0 || rope->cols % 128 || rope->cols > rows)
    return DK_ERR_INVALID;
  if (!dk_aligned(rope->cos_table, 16) || !dk_aligned(rope->sin_table, 16) || !dk_aligned(w16, 16))
    return DK_ERR_ALIGN;
  if (int e = set_side(p, side)) return e;
  p.rope_pos = rope->pos;
  p.rope_cos = rope->cos_table;
  p.rope_sin = rope->sin_table;
  p.rope_hd = rope->hd;
  p.rope_cols = rope->cols;
  if (p.M == 0) return side_alone(p.side, stream);
  p.w16 = (const f16*)w16;
  const int r = hgemm_launch<false, EPI_LINEAR>(p, nullptr, 0, stream);
  return r == kHgemmDeclined ? DK_ERR_INVALID : r;   // a shape the fused rotary form does not take
}

extern "C" int dk_h16_linear_bwd_dx_lora(const void* dy, int64_t lddy, int64_t m, const void* w16,
                                         int64_t rows, int64_t cols, const dk_lora_term* terms,
                                         int n_terms, int64_t rank, void* dx, int64_t lddx,
                                         int out_mode, void* workspace, int64_t workspace_bytes,
                                         const dk_side_dequant* side, hipStream_t stream) {
  GemmParams p = {};
  if (int e = linear_bwd_params(p, dy, lddy, m, rows, cols, terms, n_terms, rank, dx, lddx,
                                out_mode))
    return e;
  return dispatch_h16<true, EPI_LINEAR>(p, w16, workspace, workspace_bytes, side, stream);
}

extern "C" int dk_h16_linear_bwd_dx_lora_sums(const void* dy, int64_t lddy, int64_t m,
                                              const void* w16, int64_t rows, int64_t cols,
                                              const dk_lora_term* terms, int n_terms, int64_t rank,
                                              void* dx, int64_t lddx, int out_mode,
                                              void* workspace, int64_t workspace_bytes,
                                              const dk_side_dequant* side,
                                              const dk_side_lora_sums* sums, hipStream_t stream) {
  GemmParams p = {};
  if (int e = linear_bwd_params(p, dy, lddy, m, rows, cols, terms, n_terms, rank, dx, lddx,
                                out_mode))
    return e;
  CarriedSums cs;
  if (int e = set_sums(cs, sums)) return e;
  return dispatch_h16<true, EPI_LINEAR>(p, w16, workspace, workspace_bytes, side, stream, cs);
}

// ---- the allocation-free dX entry point: split-K partials in a library-owned device array

// One copy per device, allocated with the code object and held until the process ends.  In host
// code `scratch` names a host-side stand-in, never the device memory: the device address comes
// from hipGetSymbolAddress, once per device with that device current, and only that address is
// passed to kernels.
static __device__ __align__(256) uint8_t scratch[DK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's scratch array (looked up on the first call on a device,
// which must not be under stream capture: the lookup may load the code object, which a capture
// does not allow).
int scratch_on_current_device(hipStream_t stream, void** out) {
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev)) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return DK_ERR_INVALID;
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (!g_scratch_ptr[dev]) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipError_t e = hipStreamIsCapturing(stream, &cap)) return (int)e;
    if (cap != hipStreamCaptureStatusNone) return DK_ERR_CAPTURE;
    void* ptr = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch))) return (int)e;
    if (!ptr) return DK_ERR_INVALID;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" int dk_h16_linear_bwd_dx_lora_noalloc(const void* dy, int64_t lddy, int64_t m,
                                                 const void* w16, int64_t rows, int64_t cols,
                                                 const dk_lora_term* terms, int n_terms,
                                                 int64_t rank, void* dx, int64_t lddx,
                                                 int out_mode, const dk_side_dequant* side,
                                                 hipStream_t stream) {
  GemmParams p = {};
  if (int e = linear_bwd_params(p, dy, lddy, m, rows, cols, terms, n_terms, rank, dx, lddx,
                                out_mode))
    return e;
  // the partials this call's plan needs (0 without split-K), within the array's size; the
  // dispatch is given the whole array, so a fallback plan (one the 256-tile kernel declines at
  // launch, e.g. for an unaligned dx) finds room for its own partials too
  const int64_t need = dk_h16_workspace(m, rows, cols, DK_OP_LINEAR_BWD_DX);
  if (need > DK_NOALLOC_SCRATCH_BYTES) return DK_ERR_WORKSPACE;
  void* ws = nullptr;
  if (need > 0) {
    if (int e = scratch_on_current_device(stream, &ws)) return e;
  }
  return dispatch_h16<true, EPI_LINEAR>(p, w16, ws, ws ? DK_NOALLOC_SCRATCH_BYTES : 0, side,
                                        stream);
}

extern "C" int dk_h16_gateup_swiglu_fwd(const void* x, int64_t ldx, int64_t m, const void* w16,
                                        int64_t rows, int64_t cols, void* act, void* gu_out,
                                        void* workspace, int64_t workspace_bytes,
                                        const dk_side_dequant* side, hipStream_t stream) {
  GemmParams p = {};
  if (int e = gateup_params(p, x, ldx, m, rows, cols, act, gu_out)) return e;
  return dispatch_h16<false, EPI_SWIGLU_FWD>(p, w16, workspace, workspace_bytes, side, stream);
}

extern "C" int dk_h16_down_swiglu_bwd(const void* dh, int64_t lddh, int64_t m, const void* w16,
                                      int64_t rows, int64_t cols, void* gu, void* workspace,
                                      int64_t workspace_bytes, const dk_side_dequant* side,
                                      hipStream_t stream) {
  GemmParams p = {};
  if (int e = down_bwd_params(p, dh, lddh, m, rows, cols, gu)) return e;
  return dispatch_h16<true, EPI_SWIGLU_BWD>(p, w16, workspace, workspace_bytes, side, stream);
}

extern "C" int64_t dk_h16_workspace(int64_t m, int64_t rows, int64_t cols, int op) {
  if (m <= 0 || rows <= 0 || cols <= 0) return 0;
  // the 256 x 256-tile kernel's split-K partials where it takes the shape, else the plan's
  int64_t n = 0, k = 0;
  switch (op) {
    case DK_OP_LINEAR_FWD: n = rows; k = cols; break;
    case DK_OP_LINEAR_BWD_DX: n = cols; k = rows; break;
    default: return 0;
  }
  const int64_t big = hgemm_workspace(m, n, k, EPI_LINEAR, op == DK_OP_LINEAR_FWD);
  return big >= 0 ? big : plan_workspace(plan_for(m, n, k, EPI_LINEAR));
}

extern "C" int64_t dk_w4_workspace(int64_t m, const dk_nf4_weight* w, int op) {
  if (m <= 0 || !weight_ok(w)) return 0;
  switch (op) {
    case DK_OP_LINEAR_FWD: return gemm_workspace(m, w->rows, w->cols, EPI_LINEAR, true);
    case DK_OP_LINEAR_BWD_DX: return gemm_workspace(m, w->cols, w->rows, EPI_LINEAR, false);
    case DK_OP_GATEUP_SWIGLU_FWD: return gemm_workspace(m, w->rows, w->cols, EPI_SWIGLU_FWD, true);
    case DK_OP_DOWN_SWIGLU_BWD: return gemm_workspace(m, w->cols, w->rows, EPI_SWIGLU_BWD, false);
    default: return 0;
  }
}

extern "C" int64_t dk_w4_linear_workspace(int64_t m, const dk_nf4_weight* w, int backward) {
  return dk_w4_workspace(m, w, backward ? DK_OP_LINEAR_BWD_DX : DK_OP_LINEAR_FWD);
}
