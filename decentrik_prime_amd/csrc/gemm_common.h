// Parameters shared by the fused GEMM kernels (w4gemm.hip: NF4 or fp16 weights, warp-specialised
// 128-row tiles; hgemm.hip: fp16 weights, 256 x 256 tiles fed by LDS-DMA loads).
#pragma once
#include "lora_dev.h"
#include "nf4_dev.h"

namespace dk {

enum { EPI_LINEAR = 0, EPI_SWIGLU_FWD = 1, EPI_SWIGLU_BWD = 2 };

// One LoRA term of the LINEAR epilogue.  Forward: adds s * fp32(fp16(z B^T)) to output columns
// [n_begin, n_end) (B holds the rows of those columns).  Backward: adds
// (mask ? fp32(fp16(dz A)) * keep_scale : 0) to every column.
struct LoraTerm {
  const f16* z;         // [M][rank]: z (forward) or dz (backward)
  const f16* r;         // forward: B [n_end - n_begin][rank]; backward: A [rank][N]
  const uint8_t* mask;  // backward keep-mask [M][N] or null (no dropout, no scale)
  int64_t n_begin, n_end;
  float scale;          // forward: s; backward: keep_scale
};

struct GemmParams {
  const f16* a;
  int64_t lda;
  int64_t M, N, K;
  const uint8_t* packed;
  const uint8_t* qabs;
  const float* scale2;
  const float* offset2;
  const float* code2;
  const float* nf4;
  const f16* w16;       // two-phase: the weight dequantised to fp16, stored order ([N][K] NT, [K][N] NN)
  int64_t inter;        // SwiGLU: gate/up width I
  const f16* bias;      // [N] or null
  LoraTerm lora[2];     // rank-r LoRA terms added in the LINEAR epilogue, in order
  int n_lora;
  int64_t rank;
  void* out;
  int64_t ldo;
  int out_mode;
  f16* gu;              // SWIGLU_FWD: optional [M][2I] output; SWIGLU_BWD: [M][2I] in/out
  int tiles_m, tiles_n;
  int m_fastest;        // tile order: row tiles fastest (1) or column tiles fastest (0)
  int xcd_gm;           // 256-tile kernel: the 128 x 128 quarters split into a block per XCD,
                        // xcd_gm blocks along M by 8 / xcd_gm along N (0: runs of quarters)
  int splits;           // split-K factor (1: none)
  float* part;          // split-K partial tiles [tiles][splits][BM * BN] fp32
  SideDequant side;     // dequant work carried by the launch's last side.wgs workgroups
  SideSums sums;        // LoRA column sums carried by the sums.wgs workgroups before those
  // LINEAR NT only: rotary embedding of output columns [0, rope_cols) (the q and k heads of a
  // fused QKV projection) in the epilogue, before the single fp16 rounding; null: none
  const int32_t* rope_pos;   // [M] token positions
  const float* rope_cos;     // [positions][rope_hd]
  const float* rope_sin;
  int rope_hd;               // head size: two 64-column wave blocks
  int64_t rope_cols;
};

// Runs the GEMM of `p` (fp16 weight p.w16) on the 256 x 256-tile kernel when the shape suits it:
// output columns a multiple of 256, K a multiple of 64, and either at least one tile per CU, or
// (LINEAR, at least 4 row tiles, K of 4096 or more) a split-K that fills the CUs, whose fp32
// partials need hgemm_workspace bytes of `ws`, or 128 x 128 tiles that fill at least half the
// CUs.  p.side's workgroups (if any) join the launch.  Returns kHgemmDeclined without launching
// anything otherwise, a HIP error code, or 0.
constexpr int kHgemmDeclined = -1000;
// W4: the weight read as packed NF4 (p.packed, p.qabs, p.scale2, p.offset2, p.code2, p.nf4; no
// p.w16) and dequantised by each workgroup into LDS, bit-identical to the fp16 form's results.
template <bool TRANS, int EPI, bool W4 = false>
int hgemm_launch(const GemmParams& p, void* ws, int64_t ws_bytes, hipStream_t stream);
// Split-K partials the launch of that shape needs (0: no split; -1: the plan does not take the
// shape); nt: NT (W stored [N][K]).
int64_t hgemm_workspace(int64_t M, int64_t N, int64_t K, int epi, bool nt);

}  // namespace dk
