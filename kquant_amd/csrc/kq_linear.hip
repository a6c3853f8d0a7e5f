// Dense dequant-fused linear: C[M, N] = A[M, K] (bf16) x dequant(W)[N, K]^T,
// W in MXFP8 (E4M3) or MXFP4 (E2M1) with per-32 E8M0 scales, fp32
// accumulation on v_mfma_f32_32x32x16_bf16, bf16 or fp32 output.
//
// This is the A16 operand contract of kquant's MXFP8 closure oracle
// (scripts/closure_mxfp8_mlp.py:146-187: fp32 matmul over the dequantized
// weights) and of the W4A16 expert linears.
//
// Workgroup tile 256 x 256, 8 waves of 64 x 128 (2 x 4 MFMA 32x32 blocks),
// K step 64, LDS double buffered.  Weights are staged in LDS still packed
// (E4M3: 64 B per row and step, E2M1: 32 B) and expanded to bf16 per fragment.
#include "kq_dma.h"
#include "kq_gemm.h"
#include "kq_internal.h"

namespace kq {

namespace lin {
constexpr int BM = 256, BN = 256, BK = 64;
constexpr int THREADS = 512;
constexpr int A_ROW = BK * 2 + 16;                  // 144 B: bf16 row + pad
template <int FMT> constexpr int b_row() { return FMT == 0 ? 72 : 36; }  // packed row + pad
constexpr int A_BYTES = BM * A_ROW;                 // 36 KiB
template <int FMT> constexpr int b_bytes() { return BN * b_row<FMT>(); }
constexpr int S_BYTES = BN * 2;                     // 2 scale bytes per row per step
template <int FMT> constexpr int stage_bytes() { return A_BYTES + b_bytes<FMT>() + S_BYTES; }
}  // namespace lin

using gemm::bf16x8_t;
using gemm::u32x2_t;
using gemm::u32x4_t;

template <int FMT, int OUT>
__global__ __launch_bounds__(512, 1) void mx_linear_kernel(
    const uint16_t* __restrict__ a, int64_t lda, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, void* __restrict__ c, int64_t ldc, int M, int N, int K, int KB) {
  using namespace lin;
  constexpr int BROW = b_row<FMT>();
  constexpr int WBYTES = FMT == 0 ? BK : BK / 2;  // packed bytes per row per step
  extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  // A has K columns; the weights have KB (K is a multiple of KB, and A's
  // column k multiplies weight column k % KB: the split-fp32 operand).
  const int64_t kw = FMT == 0 ? KB : KB / 2;  // packed bytes per weight row
  const int64_t ks = KB / 32;                 // scale bytes per weight row

  // ---- global -> register staging
  u32x4_t ra[4], rb[2];
  uint32_t rs = 0;
  auto load = [&](int k0) {
    const int kb0 = k0 % KB;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + THREADS * i;  // 2048 chunks of 16 B
      const int row = ch >> 3, col = (ch & 7) * 8;
      const int gm = m0 + row;
      ra[i] = gm < M ? *reinterpret_cast<const u32x4_t*>(a + (int64_t)gm * lda + k0 + col)
                     : u32x4_t{0u, 0u, 0u, 0u};
    }
    constexpr int BCH = BN * WBYTES / 16;  // chunks of 16 B
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = tid + THREADS * i;
      if (ch < BCH) {
        const int row = ch / (WBYTES / 16), col = (ch % (WBYTES / 16)) * 16;
        const int gn = n0 + row;
        rb[i] = gn < N ? *reinterpret_cast<const u32x4_t*>(wq + (int64_t)gn * kw + (FMT == 0 ? kb0 : kb0 / 2) + col)
                       : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    if (tid < BN) {
      const int gn = n0 + tid;
      rs = gn < N ? *reinterpret_cast<const uint16_t*>(ws + (int64_t)gn * ks + kb0 / 32) : 0u;
    }
  };
  auto store = [&](int buf) {
    unsigned char* base = lds + buf * stage_bytes<FMT>();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ch = tid + THREADS * i;
      const int row = ch >> 3, col = (ch & 7) * 16;
      *reinterpret_cast<u32x4_t*>(base + row * A_ROW + col) = ra[i];
    }
    unsigned char* bb = base + A_BYTES;
    constexpr int BCH = BN * WBYTES / 16;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = tid + THREADS * i;
      if (ch < BCH) {
        const int row = ch / (WBYTES / 16), col = (ch % (WBYTES / 16)) * 16;
        if (FMT == 0) {
          *reinterpret_cast<u32x2_t*>(bb + row * BROW + col) = u32x2_t{rb[i][0], rb[i][1]};
          *reinterpret_cast<u32x2_t*>(bb + row * BROW + col + 8) = u32x2_t{rb[i][2], rb[i][3]};
        } else {
#pragma unroll
          for (int d = 0; d < 4; ++d) *reinterpret_cast<uint32_t*>(bb + row * BROW + col + 4 * d) = rb[i][d];
        }
      }
    }
    if (tid < BN) *reinterpret_cast<uint16_t*>(base + A_BYTES + b_bytes<FMT>() + tid * 2) = (uint16_t)rs;
  };

  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
  float16_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int frow = lane & 31, fk = lane >> 5;  // fragment row, k half (8 elements)
  const int steps = K / BK;
  load(0);
  store(0);
  __syncthreads();
  for (int s = 0; s < steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < steps) load((s + 1) * BK);
    const unsigned char* base = lds + buf * stage_bytes<FMT>();
    const unsigned char* bb = base + A_BYTES;
    const unsigned char* sb = bb + b_bytes<FMT>();
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      bf16x8_t fa[2], fb[4];
#pragma unroll
      for (int i = 0; i < 2; ++i)
        fa[i] = *reinterpret_cast<const bf16x8_t*>(base + (wm + i * 32 + frow) * A_ROW + kk * 32 + fk * 16);
      // this lane's 8 k values lie in scale block (kk * 16 + fk * 8) / 32 = kk / 2
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int row = wn + j * 32 + frow;
        const uint32_t sc = sb[row * 2 + (kk >> 1)];
        u32x2_t w;
        if (FMT == 0) {
          w = *reinterpret_cast<const u32x2_t*>(bb + row * BROW + kk * 16 + fk * 8);
        } else {
          w[0] = *reinterpret_cast<const uint32_t*>(bb + row * BROW + kk * 8 + fk * 4);
          w[1] = 0u;
        }
        fb[j] = gemm::dequant8<FMT>(w, sc);
      }
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    }
    if (s + 1 < steps) store(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: C[32x32] lane layout col = lane % 32, row = 8(r/4) + 4(lane/32) + r%4
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int gm = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * fk + (r & 3);
        const int gn = n0 + wn + j * 32 + frow;
        if (gm < M && gn < N) {
          if (OUT == 2) static_cast<float*>(c)[(int64_t)gm * ldc + gn] = acc[i][j][r];
          else static_cast<__bf16*>(c)[(int64_t)gm * ldc + gn] = (__bf16)acc[i][j][r];
        }
      }
}

// ------------------------------------------------ direct-to-LDS variant --
// Same tile (256 x 256, K step 64) and result as mx_linear_kernel, with every
// operand moved HBM -> LDS by buffer_load ... lds through a ring of three
// stages, continuing across tile boundaries: the kernel is persistent (one
// workgroup per CU, tiles t = worker, worker + G, ... in groups of
// LIN_GROUP_M row tiles with N fastest inside a group, workers of one XCD
// numbered consecutively so the 32 tiles they run together share 4 A row
// tiles and 8 weight column tiles in its L2).
//  * four waves of 128 x 128, one per SIMD: each keeps 16 32x32 accumulators
//    (256 registers, AGPRs) and runs 64 MFMAs per step, so every fragment
//    read from LDS feeds four MFMAs.  One wave per SIMD issues in order, so
//    every other instruction of a step has a fixed place between two MFMAs
//    (sched_barrier pins the order, empty asm keeps the expansions where they
//    are placed): nothing else runs while the matrix core waits.
//  * a step: k16 block 0 of the step's MFMAs (the rest of the stage in flight
//    is issued between them), the one barrier of the step (stage s + 1 has
//    landed and every wave holds all of slot s in registers, so slot s is
//    free), then blocks 1-3, between whose 48 MFMAs go the LDS reads of step
//    s + 1 (at most one per MFMA, so they do not crowd the LDS; each writes
//    its registers in place once their old value is dead, block 3's from
//    the current slot during the next step's block 0), the first direct
//    loads of stage s + 3 (into slot s) and the expansions.  A stage's
//    13 direct loads per wave (E4M3; 11 E2M1; one fewer with unit scales)
//    thus spread over two steps and are waited for one step after the last.
//  * k order: in a 64-k step, lane half f of MFMA q (0..3) takes
//    k = 32 f + 8 q + [0, 8) on both operands, so a lane's weights for the
//    step are one 16-byte chunk (E2M1) or two (E4M3) of its row, read with
//    128-bit LDS reads, under the one scale byte of block f.
//  * A rows: 128 B per stage, 16-byte chunk c of row r at slot c ^ ((r/2)%8).
//    Weight rows: 32 B (E2M1) / 64 B (E4M3) per stage, chunk c of row r at
//    slot c ^ ((r/8)%2) / c ^ ((r/4)%4).  Either way the 16 lanes of a read
//    hit 16 distinct bank groups.
//  * scales: one aligned dword per weight row per stage (four blocks, two of
//    them this step's) by 4-byte direct loads; needs KB % 128 == 0.
//  * rows past M or N read as zero (out-of-range offsets) and are not stored.
//  * split K (fp32 output only): with `slices` > 1 the work items are
//    (slice, tile), slice-major, and item (s, t) runs steps
//    [s steps / slices, (s + 1) steps / slices) of tile t into plane s of c
//    (c + s plane); the caller sums the planes.  Needs slices <= steps.
//  * UNIT: every E8M0 scale is 127 (x 1); no scale array is read.
namespace lin3 {
constexpr int NSTAGE = 3;
constexpr int A_BYTES = lin::BM * lin::BK * 2;                      // 32 KiB
template <int FMT> constexpr int w_row() { return FMT == 0 ? 64 : 32; }  // bytes per row per stage
template <int FMT> constexpr int b_bytes() { return lin::BN * w_row<FMT>(); }
constexpr int S_BYTES = lin::BN * 4;
template <int FMT> constexpr int stage() { return A_BYTES + b_bytes<FMT>() + S_BYTES; }
constexpr int LIN_GROUP_M = 4;  // row tiles per group of the tile order

// Tile tl of the grouped order -> (row tile mt, column tile nt).
__device__ __forceinline__ void tile_mn(int tl, int mtiles, int ntiles, int& mt, int& nt) {
  const int per = LIN_GROUP_M * ntiles, g = tl / per, rem = tl - g * per;
  const int gsz = min(LIN_GROUP_M, mtiles - g * LIN_GROUP_M);
  mt = g * LIN_GROUP_M + rem % gsz;
  nt = rem / gsz;
}
}  // namespace lin3

__shared__ __attribute__((aligned(16))) unsigned char lin3_lds[lin3::NSTAGE * lin3::stage<0>()];

template <int FMT, int OUT, bool UNIT = false>
__global__ __launch_bounds__(256, 1) void mx_linear_dma_kernel(
    const uint16_t* __restrict__ a, int64_t lda, uint32_t a_bytes, const uint8_t* __restrict__ wq,
    const uint8_t* __restrict__ ws, uint32_t w_bytes, uint32_t s_bytes, void* __restrict__ c,
    int64_t ldc, int M, int N, int K, int KB, int slices, int64_t plane) {
  using namespace lin3;
  using dma::i32x4_t;
  constexpr int WQ = FMT == 0 ? 4 : 2;  // weight loads per wave per stage
  constexpr int H = FMT == 0 ? 2 : 1;   // 16-byte weight chunks per row and step
  constexpr int WROW = w_row<FMT>(), STAGE = stage<FMT>(), LOADS = 8 + WQ + (UNIT ? 0 : 1);
  constexpr int BM = lin::BM, BN = lin::BN, BK = lin::BK;
  const int mtiles = (M + BM - 1) / BM, ntiles = (N + BN - 1) / BN, tiles = mtiles * ntiles;
  const int total = tiles * slices;
  const int G = gridDim.x;
  const int worker = (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8);
  if (worker >= total) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int lw = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t kw = FMT == 0 ? KB : KB / 2;
  const int64_t ks = KB / 32;
  const int steps = K / BK;
  const uint32_t lds0 = dma::lds_offset_of(lin3_lds);
  const i32x4_t a_rsrc = dma::make_rsrc(a, a_bytes);
  const i32x4_t w_rsrc = dma::make_rsrc(wq, w_bytes);
  const i32x4_t s_rsrc = dma::make_rsrc(ws, s_bytes);

  int lt = worker, ls = 0, ls_end = steps;
  uint32_t a_base = 0, w_base = 0, s_off = 0;
  int a_lim = 0, w_lim = 0;
  const uint32_t a_qstep = (uint32_t)(32 * lda * 2);
  constexpr int WSTEP = FMT == 0 ? 64 : 128;
  const uint32_t w_qstep = (uint32_t)(WSTEP * kw);
  auto set_load_tile = [&]() {
    const bool live = lt < total;
    const int sl = live ? lt / tiles : 0, tl = live ? lt - sl * tiles : 0;
    ls = (int)((int64_t)sl * steps / slices);
    ls_end = (int)((int64_t)(sl + 1) * steps / slices);
    int mt = 0, nt = 0;
    if (live) tile_mn(tl, mtiles, ntiles, mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;
    {
      const int row = 8 * lw + (lane >> 3);
      const int ch = (lane & 7) ^ ((row >> 1) & 7);
      a_lim = live ? M - m0 - row : 0;
      a_base = a_lim > 0 ? (uint32_t)((int64_t)(m0 + row) * lda * 2 + ch * 16) : 0u;
    }
    {
      const int row = FMT == 0 ? 16 * lw + (lane >> 2) : 32 * lw + (lane >> 1);
      const int ch = FMT == 0 ? (lane & 3) ^ ((row >> 2) & 3) : (lane & 1) ^ ((row >> 3) & 1);
      w_lim = live ? N - n0 - row : 0;
      w_base = w_lim > 0 ? (uint32_t)((int64_t)(n0 + row) * kw + ch * 16) : 0u;
    }
    {
      const int row = 64 * lw + lane;
      s_off = live && n0 + row < N ? (uint32_t)((int64_t)(n0 + row) * ks) : s_bytes;
    }
  };
  // load u (0-7 A, then WQ weight loads, then the scale load) of the stage at ls into slot
  auto issue_one = [&](int slot, int u) {
    const uint32_t base = lds0 + (uint32_t)(slot * STAGE);
    const int k0 = ls * BK, kb0 = k0 % KB;
    if (u < 8) {
      dma::load_to_lds16(a_rsrc, 32 * u < a_lim ? a_base + u * a_qstep + 2 * (uint32_t)k0 : a_bytes,
                         base + (uint32_t)((4 * u + lw) * 1024));
    } else if (u < 8 + WQ) {
      const int q = u - 8;
      const uint32_t wk = FMT == 0 ? (uint32_t)kb0 : (uint32_t)kb0 / 2;
      dma::load_to_lds16(w_rsrc, WSTEP * q < w_lim ? w_base + q * w_qstep + wk : w_bytes,
                         base + (uint32_t)(A_BYTES + (4 * q + lw) * 1024));
    } else if (!UNIT) {
      dma::load_to_lds4(s_rsrc, s_off >= s_bytes ? s_bytes : s_off + (uint32_t)((kb0 / 32) & ~3),
                        base + (uint32_t)(A_BYTES + b_bytes<FMT>() + lw * 256));
    }
  };
  auto issue = [&](int slot) {
#pragma unroll
    for (int u = 0; u < LOADS; ++u) issue_one(slot, u);
  };
  auto advance = [&]() {
    if (++ls == ls_end) {
      lt += G;
      set_load_tile();
    }
  };

  const int wm = (lw >> 1) * 128, wn = (lw & 1) * 128;
  const int frow = lane & 31, f = lane >> 5;
  int arow[4], axor[4], woff[4][H], soff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = wm + i * 32 + frow;
    arow[i] = row * (BK * 2);
    axor[i] = (4 * f) ^ ((row >> 1) & 7);
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = wn + j * 32 + frow;
    if (FMT == 0) {
      woff[j][0] = A_BYTES + row * WROW + 16 * ((2 * f) ^ ((row >> 2) & 3));
      woff[j][H - 1] = A_BYTES + row * WROW + 16 * ((2 * f + 1) ^ ((row >> 2) & 3));
    } else {
      woff[j][0] = A_BYTES + row * WROW + 16 * (f ^ ((row >> 3) & 1));
    }
    soff[j] = A_BYTES + b_bytes<FMT>() + row * 4;  // the row's scale dword
  }

  // one step's fragments: weight chunks, scale dwords (four blocks of the
  // row; this lane's byte is picked when the step runs) and A fragments
  constexpr int NR = 4 * H + (UNIT ? 0 : 4) + 16;  // LDS reads per step
  u32x4_t wv[4][H];
  uint32_t scw[4];
  bf16x8_t fa[4][4];
  // read r of a step from slot st: weight chunks, then scale dwords, then A fragments
  auto read_one = [&](const unsigned char* st, int r, u32x4_t (&w)[4][H], uint32_t (&sw)[4], bf16x8_t (&a)[4][4]) {
    if (r < 4 * H) {
      w[r / H][r % H] = *reinterpret_cast<const u32x4_t*>(st + woff[r / H][r % H]);
    } else if (!UNIT && r < 4 * H + 4) {
      sw[r - 4 * H] = *reinterpret_cast<const uint32_t*>(st + soff[r - 4 * H]);
    } else {
      const int e = r - (NR - 16), q = e >> 2, i = e & 3;
      a[q][i] = *reinterpret_cast<const bf16x8_t*>(st + arow[i] + 16 * (q ^ axor[i]));
    }
  };
  auto expand1 = [&](const u32x4_t (&w4)[4][H], int q, int j, const uint32_t (&sc)[4]) -> bf16x8_t {
    u32x2_t w;
    if (FMT == 0) w = u32x2_t{w4[j][q >> 1][2 * (q & 1)], w4[j][q >> 1][2 * (q & 1) + 1]};
    else w = u32x2_t{w4[j][0][q], 0u};
    return gemm::dequant8<FMT>(w, sc[j]);
  };
  auto scale_bytes = [&](const uint32_t (&sw)[4], int kb, uint32_t (&sc)[4]) {
    const int sh = 8 * ((kb >> 5) & 3) + 8 * f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      sc[j] = UNIT ? 127u : (sw[j] >> sh) & 0xffu;
      asm volatile("" : "+v"(sc[j]));  // computed here, not sunk to its first use
    }
  };
  // an expansion computed where it is placed, not sunk to its first use
  auto pinned = [](bf16x8_t v) -> bf16x8_t {
    asm volatile("" : "+v"(v));
    return v;
  };
  // The loads of a stage are split: LA of them among the MFMAs of k16 block
  // 3 of one step, the rest among those of block 0 of the next, so the four
  // waves' direct loads spread over the whole step.
  constexpr int LA = LOADS > 7 ? 7 : LOADS;
  int lslot = 0;  // ring slot of the stage at ls
  auto next_stage = [&]() {
    advance();
    lslot = lslot == 2 ? 0 : lslot + 1;
  };

  set_load_tile();
  issue(0);
  next_stage();
  issue(1);
  next_stage();
  dma::wait_and_barrier<LOADS>();  // stage 0 landed
#pragma unroll
  for (int r = 0; r < NR; ++r) read_one(lin3_lds, r, wv, scw, fa);
#pragma unroll
  for (int u = 0; u < LA; ++u) issue_one(lslot, u);
  uint32_t sc[4];
  bf16x8_t fb0[4];
  {
    const int s0 = worker < total ? (int)((int64_t)(worker / tiles) * steps / slices) : 0;
    scale_bytes(scw, (int)((int64_t)s0 * BK % KB), sc);
#pragma unroll
    for (int j = 0; j < 4; ++j) fb0[j] = expand1(wv, 0, j, sc);
  }
  int cslot = 0;
  for (int t = worker; t < total; t += G) {
    const int sl = t / tiles, tl = t - sl * tiles;
    int mt, nt;
    tile_mn(tl, mtiles, ntiles, mt, nt);
    const int s_begin = (int)((int64_t)sl * steps / slices), s_end = (int)((int64_t)(sl + 1) * steps / slices);
    const int m0 = mt * BM, n0 = nt * BN;
    const bool active = m0 + wm < M && n0 + wn < N;
    // k of the first step of the next work item (its scale bytes are picked at this item's last step)
    const int kb_next_item = t + G < total ? (int)((int64_t)((t + G) / tiles) * steps / slices * BK % KB) : 0;
    float16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    int kb = (int)((int64_t)s_begin * BK % KB);  // k of the step within its scale row
    // One wave per SIMD issues in order, so every load, LDS read and expansion
    // has a fixed place between two MFMAs (sched_barrier pins the order): the
    // matrix core never waits behind a run of other instructions, and the
    // LDS reads of the next step (at most one per MFMA) spread over the 48
    // MFMAs after the barrier instead of crowding the LDS.
    for (int s = s_begin; s < s_end; ++s) {
      kb = kb + BK == KB ? 0 : kb + BK;
      const unsigned char* cst = lin3_lds + cslot * STAGE;
      bf16x8_t fb1[4], fb2[4], fb3[4];
      // k16 block 0 (expanded at the end of the previous step); the rest of
      // the stage in flight; expansion of block 1
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[0][m >> 2], fb0[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
        if (!(m & 1) && m / 2 < LOADS - LA) issue_one(lslot, LA + m / 2);
        if ((m & 1) && m / 2 < 4) fb1[m / 2] = pinned(expand1(wv, 1, m / 2, sc));
        if ((m & 1) && m >= 9) read_one(cst, NR - 16 + 12 + (m - 9) / 2, wv, scw, fa);  // A block 3
        __builtin_amdgcn_sched_barrier(0);
      }
      next_stage();
      // stage s + 1 landed; every wave has every fragment of slot s in registers
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): no read of slot s is still in flight
      dma::wait_and_barrier<LOADS>();
      __builtin_amdgcn_sched_barrier(0);
      const int nslot = cslot == 2 ? 0 : cslot + 1;
      const unsigned char* nst = lin3_lds + nslot * STAGE;
      const int kb_next = s + 1 < s_end ? kb : kb_next_item;
      // slot m (0-47) of the MFMAs of blocks 1-3.  The reads of step s + 1
      // (this item's or the next one's) write the registers in place, each
      // once its old value is dead: A block 0 at once, block 1 after its
      // MFMAs (m >= 16), the weight chunks and scale dwords after the last
      // expansion (m >= 24), block 2 after its MFMAs (m >= 32); block 3 is
      // read from this slot during the next step's block 0.  Between them the
      // expansions of blocks 2 and 3, the first loads of stage s + 3 (into
      // slot s, free since the barrier), then the scale bytes and block-0
      // expansion of step s + 1.
      auto slot_work = [&](int m) {
        if (m < 8 && !(m & 1)) read_one(nst, NR - 16 + m / 2, wv, scw, fa);
        if (m >= 16 && m < 24 && !(m & 1)) read_one(nst, NR - 16 + 4 + (m - 16) / 2, wv, scw, fa);
        if (m >= 24 && m < 24 + 4 * H) read_one(nst, m - 24, wv, scw, fa);
        if (!UNIT && m >= 32 && m < 36) read_one(nst, 4 * H + (m - 32), wv, scw, fa);
        if (m >= 36 && m < 40) read_one(nst, NR - 16 + 8 + (m - 36), wv, scw, fa);
        if (m < 8 && (m & 1)) fb2[m / 2] = pinned(expand1(wv, 2, m / 2, sc));
        if (m >= 16 && m < 24 && (m & 1)) fb3[(m - 16) / 2] = pinned(expand1(wv, 3, (m - 16) / 2, sc));
        if (m >= 32 && !(m & 1) && (m - 32) / 2 < LA) issue_one(lslot, (m - 32) / 2);
        if (m == 43) scale_bytes(scw, kb_next, sc);
        if (m >= 44) fb0[m - 44] = pinned(expand1(wv, 0, m - 44, sc));
      };
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[1][m >> 2], fb1[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
        slot_work(m);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[2][m >> 2], fb2[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
        slot_work(16 + m);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        acc[m >> 2][m & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[3][m >> 2], fb3[m & 3], acc[m >> 2][m & 3], 0, 0, 0);
        slot_work(32 + m);
        __builtin_amdgcn_sched_barrier(0);
      }
      cslot = nslot;
    }

    if (active) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int gm = m0 + wm + i * 32 + 8 * (r >> 2) + 4 * f + (r & 3);
            const int gn = n0 + wn + j * 32 + frow;
            if (gm < M && gn < N) {
              if (OUT == 2) static_cast<float*>(c)[sl * plane + (int64_t)gm * ldc + gn] = acc[i][j][r];
              else static_cast<__bf16*>(c)[(int64_t)gm * ldc + gn] = (__bf16)acc[i][j][r];
            }
          }
    }
  }
  __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));  // no load may land after the workgroup ends
}

// ------------------------------------------- MXFP8 x MXFP8 (A8W8) --
// C[M, N] = dequant(A)[M, K] x dequant(W)[N, K]^T with both operands MXFP8
// (E4M3 bytes, one E8M0 byte per 32 along K): the operand contract of
// kquant's production MXFP8 linear, which quantizes its input rows before
// the product (scripts/closure_mxfp8_mlp.py:146-160, :172-177).  One
// v_mfma_scale_f32_32x32x64_f8f6f4 per 32x32 block and 64-k step multiplies
// the E4M3 bytes with their E8M0 bytes as they are.  Lane (m, g) of a
// 32x32x64 operand holds row m and byte i at k = 32 (i / 16) + 16 g + i % 16
// (16-byte chunks g and 2 + g of the row's 64 k) and gives the scale of its
// row's block g (checked with an in-bounds one-wave probe).
//  * persistent, tiles of 256 x 256 in mx_linear_dma_kernel's grouped order,
//    workers of one XCD numbered consecutively; 8 waves of 64 x 128 (2 x 4
//    blocks) as two ping-pong groups: group 0 issues every direct load and
//    leads, group 1 runs half a step behind; a step (64 k) is a memory phase
//    (all LDS reads of the step into registers) and a compute phase (8
//    MFMAs).
//  * two LDS stages of 128 k (double buffered; a stage is two steps): per
//    stage the A and W tiles, 256 rows x 128 B each, so every direct load
//    fetches whole 128-byte lines (8 rows x 128 B per instruction), 16-byte
//    chunk c of row r at slot c ^ ((r / 2) % 8) (the 16 lanes of a 128-bit
//    read hit 16 distinct bank groups); and the stage's scale dwords of both
//    operands, read from scale planes transposed to [K / 128][rows] dwords
//    (the four blocks of a row's 128 k), 1 KiB contiguous per operand.
//    Fetching half lines, or one 4-byte scale per row, made this kernel's
//    direct loads issue 2-4x more line requests than bytes need, which
//    bounded it (measured: 376 us of loads alone at cfg2; 139 us for twice
//    the bytes in whole lines without per-row scale dwords).
//  * rows past M or N read as zero (out-of-range offsets) and are not stored.
namespace lin8 {
constexpr int BK = 64, SK = 128;             // MFMA step, LDS stage
constexpr int OP_BYTES = 256 * SK;           // one operand tile per stage
constexpr int S_OFF = 2 * OP_BYTES;          // A scale dwords, then W's
constexpr int STAGE = 2 * OP_BYTES + 2 * 1024;
constexpr int LOADS = 8 + 8 + 1 + 1;         // direct loads per loading wave per stage
}  // namespace lin8

__shared__ __attribute__((aligned(16))) unsigned char lin8_lds[2 * lin8::STAGE];

typedef int i32x8_t __attribute__((ext_vector_type(8)));

template <int OUT>
__global__ __launch_bounds__(512, 1) void mx_linear_a8_kernel(
    const uint8_t* __restrict__ aq, int64_t lda, uint32_t a_bytes, const uint32_t* __restrict__ ast,
    uint32_t ast_bytes, const uint8_t* __restrict__ wq, uint32_t w_bytes, const uint32_t* __restrict__ wst,
    uint32_t wst_bytes, void* __restrict__ c, int64_t ldc, int M, int N, int K, int MS, int NS) {
  using namespace lin8;
  using dma::i32x4_t;
  constexpr int BM = lin::BM, BN = lin::BN;
  const int mtiles = (M + BM - 1) / BM, ntiles = (N + BN - 1) / BN, total = mtiles * ntiles;
  const int G = gridDim.x;
  const int worker = (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8);
  if (worker >= total) return;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool g0 = wave < 4;
  const int lw = wave & 3;
  const int stages = K / SK, steps = K / BK;
  const uint32_t lds0 = dma::lds_offset_of(lin8_lds);
  const i32x4_t a_rsrc = dma::make_rsrc(aq, a_bytes), w_rsrc = dma::make_rsrc(wq, w_bytes);
  const i32x4_t as_rsrc = dma::make_rsrc(ast, ast_bytes), ws_rsrc = dma::make_rsrc(wst, wst_bytes);

  // ---- load side: load q (0..7) of wave lw fills the 8-row piece 4q + lw
  // of both tiles (1 KiB each); lane l fetches row 8 (4q + lw) + l / 8,
  // slot l % 8, i.e. logical chunk (l % 8) ^ ((row / 2) % 8).  Scale dwords:
  // lane l of wave lw carries row 64 lw + l of the transposed planes
  // (MS / NS rows per 128-k chunk).
  int lt = worker, ls = 0;
  const int prow = 8 * lw + (lane >> 3);  // + 32 q
  const int pch = (lane & 7) ^ ((prow >> 1) & 7);
  uint32_t a_base = 0, w_base = 0, as_off = 0, ws_off = 0;
  int a_lim = 0, w_lim = 0;
  const uint32_t a_qstep = (uint32_t)(32 * lda), w_qstep = (uint32_t)(32 * K);
  auto set_load_tile = [&]() {
    const bool live = lt < total;
    int mt = 0, nt = 0;
    if (live) lin3::tile_mn(lt, mtiles, ntiles, mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;
    a_lim = live ? M - m0 - prow : 0;
    a_base = a_lim > 0 ? (uint32_t)((int64_t)(m0 + prow) * lda + 16 * pch) : 0u;
    w_lim = live ? N - n0 - prow : 0;
    w_base = w_lim > 0 ? (uint32_t)((int64_t)(n0 + prow) * K + 16 * pch) : 0u;
    const int srow = 64 * lw + lane;
    as_off = live && m0 + srow < M ? (uint32_t)(m0 + srow) * 4u : ast_bytes;
    ws_off = live && n0 + srow < N ? (uint32_t)(n0 + srow) * 4u : wst_bytes;
  };
  auto issue = [&](int slot) {
    const uint32_t base = lds0 + (uint32_t)(slot * STAGE);
    const uint32_t k0 = (uint32_t)(ls * SK);
#pragma unroll
    for (int q = 0; q < 8; ++q)
      dma::load_to_lds16(a_rsrc, 32 * q < a_lim ? a_base + q * a_qstep + k0 : a_bytes,
                         base + (uint32_t)((4 * q + lw) * 1024));
#pragma unroll
    for (int q = 0; q < 8; ++q)
      dma::load_to_lds16(w_rsrc, 32 * q < w_lim ? w_base + q * w_qstep + k0 : w_bytes,
                         base + (uint32_t)(OP_BYTES + (4 * q + lw) * 1024));
    dma::load_to_lds4(as_rsrc, as_off >= ast_bytes ? ast_bytes : as_off + (uint32_t)ls * (uint32_t)MS * 4u,
                      base + (uint32_t)(S_OFF + lw * 256));
    dma::load_to_lds4(ws_rsrc, ws_off >= wst_bytes ? wst_bytes : ws_off + (uint32_t)ls * (uint32_t)NS * 4u,
                      base + (uint32_t)(S_OFF + 1024 + lw * 256));
  };
  auto advance = [&]() {
    if (++ls == stages) {
      ls = 0;
      lt += G;
      set_load_tile();
    }
  };

  // ---- compute side: fragment offsets of step half h (k 64 h .. 64 h + 63 of the stage)
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 128;
  const int fr = lane & 31, fg = lane >> 5;
  int aoff[2][2][2], woff[2][4][2], asb[2], wsb[4];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r = wm + 32 * i + fr, sw = (r >> 1) & 7;
      aoff[h][i][0] = r * SK + 16 * ((4 * h + fg) ^ sw);
      aoff[h][i][1] = r * SK + 16 * ((4 * h + 2 + fg) ^ sw);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = wn + 32 * j + fr, sw = (r >> 1) & 7;
      woff[h][j][0] = OP_BYTES + r * SK + 16 * ((4 * h + fg) ^ sw);
      woff[h][j][1] = OP_BYTES + r * SK + 16 * ((4 * h + 2 + fg) ^ sw);
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) asb[i] = S_OFF + 4 * (wm + 32 * i + fr) + fg;
#pragma unroll
  for (int j = 0; j < 4; ++j) wsb[j] = S_OFF + 1024 + 4 * (wn + 32 * j + fr) + fg;

  if (g0) {
    set_load_tile();
    issue(0);
    advance();
  } else {
    __builtin_amdgcn_s_barrier();  // group 1 starts half a step behind
  }
  int cslot = 0;
  for (int t = worker; t < total; t += G) {
    int mt, nt;
    lin3::tile_mn(t, mtiles, ntiles, mt, nt);
    const int m0 = mt * BM, n0 = nt * BN;
    const bool active = m0 + wm < M && n0 + wn < N;
    float16_t acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    for (int s = 0; s < steps; ++s) {
      const int h = s & 1;
      if (g0) {
        if (h == 0) {
          // stage s / 2 landed (the only one in flight); both groups are done
          // reading the other slot, which now takes the next stage
          dma::wait_and_barrier<0>();
          issue(cslot ^ 1);
          advance();
        } else {
          asm volatile("" ::: "memory");
          __builtin_amdgcn_s_barrier();
          asm volatile("" ::: "memory");
        }
      } else {
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
      }
      // memory phase
      gemm::u32x4_t av[2][2], wv[4][2];
      uint32_t sa[2], sw[4];
      if (active) {
        const unsigned char* st = lin8_lds + cslot * STAGE;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          av[i][0] = *reinterpret_cast<const gemm::u32x4_t*>(st + (h ? aoff[1][i][0] : aoff[0][i][0]));
          av[i][1] = *reinterpret_cast<const gemm::u32x4_t*>(st + (h ? aoff[1][i][1] : aoff[0][i][1]));
          sa[i] = st[asb[i] + 2 * h];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          wv[j][0] = *reinterpret_cast<const gemm::u32x4_t*>(st + (h ? woff[1][j][0] : woff[0][j][0]));
          wv[j][1] = *reinterpret_cast<const gemm::u32x4_t*>(st + (h ? woff[1][j][1] : woff[0][j][1]));
          sw[j] = st[wsb[j] + 2 * h];
        }
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      // compute phase
      if (active) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const i32x8_t b8{(int)wv[j][0][0], (int)wv[j][0][1], (int)wv[j][0][2], (int)wv[j][0][3],
                           (int)wv[j][1][0], (int)wv[j][1][1], (int)wv[j][1][2], (int)wv[j][1][3]};
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            const i32x8_t a8{(int)av[i][0][0], (int)av[i][0][1], (int)av[i][0][2], (int)av[i][0][3],
                             (int)av[i][1][0], (int)av[i][1][1], (int)av[i][1][2], (int)av[i][1][3]};
            acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8, b8, acc[i][j], 0, 0, 0, (int)sa[i],
                                                                        0, (int)sw[j]);
          }
        }
      }
      if (h) cslot ^= 1;
    }

    if (active) {
      // D (32x32): lane holds column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int gm = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * fg + (r & 3);
            const int gn = n0 + wn + 32 * j + fr;
            if (gm < M && gn < N) {
              if (OUT == 2) static_cast<float*>(c)[(int64_t)gm * ldc + gn] = acc[i][j][r];
              else static_cast<__bf16*>(c)[(int64_t)gm * ldc + gn] = (__bf16)acc[i][j][r];
            }
          }
    }
  }
  if (g0) __builtin_amdgcn_s_barrier();  // matches group 1's first barrier
  __builtin_amdgcn_s_waitcnt(dma::waitcnt_vm(0));  // no load may land after the workgroup ends
}

// Scale plane [rows, K / 32] bytes -> [K / 128][rows] dwords (the four
// blocks of each row's 128-k window), the layout mx_linear_a8_kernel loads a
// stage's scales from.  Dword (r, c) of the input is bytes 4c .. 4c + 3 of row r.
__global__ __launch_bounds__(256) void scale_dwords_t_kernel(const uint32_t* __restrict__ in, int64_t rows,
                                                             int64_t chunks, uint32_t* __restrict__ out) {
  __shared__ uint32_t tile[32][33];
  const int64_t r0 = (int64_t)blockIdx.x * 32, c0 = (int64_t)blockIdx.y * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = r0 + ty + 8 * i, cc = c0 + tx;
    tile[ty + 8 * i][tx] = r < rows && cc < chunks ? in[r * chunks + cc] : 0u;
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t cc = c0 + ty + 8 * i, r = r0 + tx;
    if (r < rows && cc < chunks) out[cc * rows + r] = tile[tx][ty + 8 * i];
  }
}

// Exact three-term bf16 split of fp32 A: a = a0 + a1 + a2 (each step keeps
// the next 8 significant bits and leaves an exactly representable residual),
// written as row [a0 | a1 | a2] of a [rows, 3k] bf16 matrix.  Four columns
// per thread.
__global__ __launch_bounds__(256) void split3_bf16_kernel(const float* __restrict__ a, int64_t lda,
                                                          int64_t rows, int64_t k,
                                                          uint16_t* __restrict__ out) {
  const int64_t q = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = k / 4;
  if (q >= rows * per_row) return;
  const int64_t r = q / per_row, c = (q - r * per_row) * 4;
  const float4_t x = *reinterpret_cast<const float4_t*>(a + r * lda + c);
  uint32_t t0[2], t1[2], t2[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float h0[2], h1[2], h2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float v = x[2 * h + j];
      h0[j] = (float)(__bf16)v;
      const float r1 = v - h0[j];
      h1[j] = (float)(__bf16)r1;
      h2[j] = r1 - h1[j];
    }
    t0[h] = f32x2_to_bf16x2_bits(h0[0], h0[1]);
    t1[h] = f32x2_to_bf16x2_bits(h1[0], h1[1]);
    t2[h] = f32x2_to_bf16x2_bits(h2[0], h2[1]);
  }
  uint16_t* o = out + r * 3 * k + c;
  *reinterpret_cast<gemm::u32x2_t*>(o) = gemm::u32x2_t{t0[0], t0[1]};
  *reinterpret_cast<gemm::u32x2_t*>(o + k) = gemm::u32x2_t{t1[0], t1[1]};
  *reinterpret_cast<gemm::u32x2_t*>(o + 2 * k) = gemm::u32x2_t{t2[0], t2[1]};
}

}  // namespace kq

using namespace kq;

// Direct-to-LDS path: needs 4-byte aligned scale rows (KB % 128 == 0, scale
// pointer 4-byte aligned); operands larger than one 32-bit buffer range are
// cut into row chunks of M and N.
template <int FMT, int OUT, bool UNIT = false>
static hipError_t launch_linear_dma(const uint16_t* a, int64_t lda, const uint8_t* wq,
                                    const uint8_t* ws, void* c, int64_t ldc, int M, int N, int K,
                                    int KB, hipStream_t st, int slices = 1, int64_t plane = 0) {
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int64_t kw = FMT == 0 ? KB : KB / 2, ks = KB / 32;
  const int64_t m_chunk = (int64_t)(dma::MAX_RANGE / (uint64_t)(lda * 2)) / lin::BM * lin::BM;
  const int64_t n_chunk = (int64_t)(dma::MAX_RANGE / (uint64_t)kw) / lin::BN * lin::BN;
  for (int64_t m0 = 0; m0 < M; m0 += m_chunk) {
    const int mc = (int)(M - m0 < m_chunk ? M - m0 : m_chunk);
    for (int64_t n0 = 0; n0 < N; n0 += n_chunk) {
      const int nc = (int)(N - n0 < n_chunk ? N - n0 : n_chunk);
      const int tiles = ((mc + lin::BM - 1) / lin::BM) * ((nc + lin::BN - 1) / lin::BN) * slices;
      int grid = cus / 8 * 8 > 0 ? cus / 8 * 8 : 8;
      if (grid > (tiles + 7) / 8 * 8) grid = (tiles + 7) / 8 * 8;
      void* cp = OUT == 2 ? (void*)(static_cast<float*>(c) + m0 * ldc + n0)
                          : (void*)(static_cast<uint16_t*>(c) + m0 * ldc + n0);
      mx_linear_dma_kernel<FMT, OUT, UNIT><<<grid, 256, 0, st>>>(
          a + m0 * lda, lda, (uint32_t)(mc * lda * 2), wq + n0 * kw, ws + n0 * ks,
          (uint32_t)(nc * kw), (uint32_t)(nc * ks), cp, ldc, mc, nc, K, KB, slices, plane);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

// MXFP8 x MXFP8 launch: both scale planes are first transposed into the
// workspace ([K / 128][rows] dwords); operands larger than one 32-bit buffer
// range are cut into row chunks of M and N, each with its own plane rows.
// Needs K % 128 == 0, lda % 16 == 0, 16-byte aligned E4M3 operands and
// 4-byte aligned scale rows of K / 32 bytes.
static int64_t a8_scale_plane_bytes(int64_t rows, int64_t k) { return (rows * (k / 32) + 255) / 256 * 256; }

template <int OUT>
static hipError_t launch_linear_a8(const uint8_t* aq, const uint8_t* as, int64_t lda, const uint8_t* wq,
                                   const uint8_t* ws, void* c, int64_t ldc, int M, int N, int K, void* workspace,
                                   hipStream_t st) {
  int dev = 0, cus = 0;
  hipError_t e = st ? hipStreamGetDevice(st, &dev) : hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int64_t chunks = K / 128;
  uint32_t* ast = static_cast<uint32_t*>(workspace);
  uint32_t* wst = reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + a8_scale_plane_bytes(M, K));
  scale_dwords_t_kernel<<<dim3((unsigned)((M + 31) / 32), (unsigned)((chunks + 31) / 32)), 256, 0, st>>>(
      reinterpret_cast<const uint32_t*>(as), M, chunks, ast);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  scale_dwords_t_kernel<<<dim3((unsigned)((N + 31) / 32), (unsigned)((chunks + 31) / 32)), 256, 0, st>>>(
      reinterpret_cast<const uint32_t*>(ws), N, chunks, wst);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int64_t m_chunk = (int64_t)(dma::MAX_RANGE / (uint64_t)lda) / lin::BM * lin::BM;
  const int64_t n_chunk = (int64_t)(dma::MAX_RANGE / (uint64_t)K) / lin::BN * lin::BN;
  for (int64_t m0 = 0; m0 < M; m0 += m_chunk) {
    const int mc = (int)(M - m0 < m_chunk ? M - m0 : m_chunk);
    for (int64_t n0 = 0; n0 < N; n0 += n_chunk) {
      const int nc = (int)(N - n0 < n_chunk ? N - n0 : n_chunk);
      const int tiles = ((mc + lin::BM - 1) / lin::BM) * ((nc + lin::BN - 1) / lin::BN);
      int grid = cus / 8 * 8 > 0 ? cus / 8 * 8 : 8;
      if (grid > (tiles + 7) / 8 * 8) grid = (tiles + 7) / 8 * 8;
      void* cp = OUT == 2 ? (void*)(static_cast<float*>(c) + m0 * ldc + n0)
                          : (void*)(static_cast<uint16_t*>(c) + m0 * ldc + n0);
      // the chunk's rows of each transposed plane start at row m0 / n0 of every
      // 128-k chunk; its range reaches the last chunk's rows
      const uint64_t ast_bytes = (uint64_t)((chunks - 1) * M + mc) * 4, wst_bytes = (uint64_t)((chunks - 1) * N + nc) * 4;
      mx_linear_a8_kernel<OUT><<<grid, lin::THREADS, 0, st>>>(
          aq + m0 * lda, lda, (uint32_t)(mc * lda), ast + m0, (uint32_t)ast_bytes, wq + n0 * K,
          (uint32_t)(nc * K), wst + n0, (uint32_t)wst_bytes, cp, ldc, mc, nc, K, M, N);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  }
  return hipSuccess;
}

template <int FMT, int OUT>
static hipError_t launch_linear(const uint16_t* a, int64_t lda, const uint8_t* wq, const uint8_t* ws,
                                void* c, int64_t ldc, int M, int N, int K, int KB, hipStream_t st) {
  if (KB % 128 == 0 && !kq_misaligned(ws, 4) && (uint64_t)lda * 2 * lin::BM <= dma::MAX_RANGE &&
      (uint64_t)(FMT == 0 ? KB : KB / 2) * lin::BN <= dma::MAX_RANGE)
    return launch_linear_dma<FMT, OUT>(a, lda, wq, ws, c, ldc, M, N, K, KB, st);
  const size_t lds = 2 * (size_t)lin::stage_bytes<FMT>();
  auto kern = mx_linear_kernel<FMT, OUT>;
  hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid((N + lin::BN - 1) / lin::BN, (M + lin::BM - 1) / lin::BM);
  kern<<<grid, lin::THREADS, lds, st>>>(a, lda, wq, ws, c, ldc, M, N, K, KB);
  return hipGetLastError();
}

namespace kq {

int mx_linear_slices(int64_t m, int64_t n, int64_t k_steps) {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    return 1;
  const int64_t tiles = ((m + lin::BM - 1) / lin::BM) * ((n + lin::BN - 1) / lin::BN);
  if (tiles <= 0 || 2 * tiles > cus) return 1;
  int64_t sl = cus / tiles;
  if (sl > k_steps / 8) sl = k_steps / 8;
  if (sl > 16) sl = 16;
  return sl < 1 ? 1 : (int)sl;
}

bool mx_linear_planes_ok(int64_t lda, int64_t kb) {
  return kb % 128 == 0 && (uint64_t)lda * 2 * lin::BM <= dma::MAX_RANGE && (uint64_t)kb * lin::BN <= dma::MAX_RANGE;
}

hipError_t mx_linear_planes_unit(const uint16_t* a, int64_t lda, const uint8_t* wq, float* c, int64_t ldc,
                                 int64_t plane, int m, int n, int k, int kb, int slices, hipStream_t st) {
  return launch_linear_dma<0, 2, true>(a, lda, wq, nullptr, c, ldc, m, n, k, kb, st, slices, plane);
}

hipError_t split3_rows(const float* a, int64_t lda, int64_t m, int64_t k, uint16_t* out, hipStream_t st) {
  const int64_t quads = m * (k / 4);
  split3_bf16_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, st>>>(a, lda, m, k, out);
  return hipGetLastError();
}

}  // namespace kq

extern "C" int kq_mx_linear(int w_fmt, const void* a, int64_t lda, const void* w_q,
                            const uint8_t* w_scale, int64_t m, int64_t n, int64_t k,
                            int out_dtype, void* c, int64_t ldc, void* stream) {
  if (w_fmt != KQ_FMT_MXFP8_E4M3 && w_fmt != KQ_FMT_MXFP4_E2M1)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear: unknown weight format %d", w_fmt);
  if (out_dtype != KQ_DT_BF16 && out_dtype != KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear: output dtype must be bf16 or f32");
  if (m < 0 || n < 0 || k <= 0 || k % 64 != 0 || lda < k || lda % 8 != 0 || ldc < n)
    return kq_fail(KQ_ERR_INVALID,
                   "kq_mx_linear: need k %% 64 == 0, lda >= k, lda %% 8 == 0, ldc >= n "
                   "(m=%lld n=%lld k=%lld lda=%lld ldc=%lld)",
                   (long long)m, (long long)n, (long long)k, (long long)lda, (long long)ldc);
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2)
    return kq_fail(KQ_ERR_LIMIT, "kq_mx_linear: dimension too large");
  if (kq_misaligned(a, 16) || kq_misaligned(w_q, 16) || kq_misaligned(w_scale, 2))
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear: a and w_q must be 16-byte aligned");
  if (m == 0 || n == 0) return KQ_OK;
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* ap = (const uint16_t*)a;
  const uint8_t* wp = (const uint8_t*)w_q;
  hipError_t e;
  if (w_fmt == KQ_FMT_MXFP8_E4M3)
    e = out_dtype == KQ_DT_BF16 ? launch_linear<0, 0>(ap, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, (int)k, st)
                                : launch_linear<0, 2>(ap, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, (int)k, st);
  else
    e = out_dtype == KQ_DT_BF16 ? launch_linear<1, 0>(ap, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, (int)k, st)
                                : launch_linear<1, 2>(ap, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, (int)k, st);
  return kq_check_launch(e, "kq_mx_linear");
}

extern "C" int64_t kq_mx_linear_f32_workspace_size(int64_t m, int64_t k) {
  if (m < 0 || k < 0) return -1;
  return m * 3 * k * 2;
}

extern "C" int kq_mx_linear_f32(int w_fmt, const float* a, int64_t lda, const void* w_q,
                                const uint8_t* w_scale, int64_t m, int64_t n, int64_t k, float* c,
                                int64_t ldc, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (w_fmt != KQ_FMT_MXFP8_E4M3 && w_fmt != KQ_FMT_MXFP4_E2M1)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear_f32: unknown weight format %d", w_fmt);
  if (m < 0 || n < 0 || k <= 0 || k % 64 != 0 || lda < k || lda % 4 != 0 || ldc < n)
    return kq_fail(KQ_ERR_INVALID,
                   "kq_mx_linear_f32: need k %% 64 == 0, lda >= k, lda %% 4 == 0, ldc >= n "
                   "(m=%lld n=%lld k=%lld lda=%lld ldc=%lld)",
                   (long long)m, (long long)n, (long long)k, (long long)lda, (long long)ldc);
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || 3 * k > INT32_MAX / 2)
    return kq_fail(KQ_ERR_LIMIT, "kq_mx_linear_f32: dimension too large");
  if (workspace_bytes < m * 3 * k * 2)
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear_f32: workspace needs %lld bytes",
                   (long long)(m * 3 * k * 2));
  if (kq_misaligned(a, 16) || kq_misaligned(w_q, 16) || kq_misaligned(w_scale, 2) ||
      kq_misaligned(workspace, 16))
    return kq_fail(KQ_ERR_INVALID, "kq_mx_linear_f32: a, w_q and workspace must be 16-byte aligned");
  if (m == 0 || n == 0) return KQ_OK;
  hipStream_t st = (hipStream_t)stream;
  uint16_t* a3 = static_cast<uint16_t*>(workspace);
  const int64_t quads = m * (k / 4);
  split3_bf16_kernel<<<(unsigned)((quads + 255) / 256), 256, 0, st>>>(a, lda, m, k, a3);
  if (int rc = kq_check_launch(hipGetLastError(), "kq_mx_linear_f32")) return rc;
  const uint8_t* wp = (const uint8_t*)w_q;
  const hipError_t e =
      w_fmt == KQ_FMT_MXFP8_E4M3
          ? launch_linear<0, 2>(a3, 3 * k, wp, w_scale, c, ldc, (int)m, (int)n, (int)(3 * k), (int)k, st)
          : launch_linear<1, 2>(a3, 3 * k, wp, w_scale, c, ldc, (int)m, (int)n, (int)(3 * k), (int)k, st);
  return kq_check_launch(e, "kq_mx_linear_f32");
}

static int check_linear_mx(const char* fn, int a_fmt, int w_fmt, int64_t lda, int64_t m, int64_t n, int64_t k,
                           int out_dtype, int64_t ldc) {
  if (a_fmt != KQ_FMT_MXFP8_E4M3 || w_fmt != KQ_FMT_MXFP8_E4M3)
    return kq_fail(KQ_ERR_INVALID, "%s: only MXFP8 (E4M3) x MXFP8 (E4M3) operands (a_fmt=%d, w_fmt=%d)", fn, a_fmt,
                   w_fmt);
  if (out_dtype != KQ_DT_BF16 && out_dtype != KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "%s: output dtype must be bf16 or f32", fn);
  if (m < 0 || n < 0 || k <= 0 || k % 128 != 0 || lda < k || lda % 16 != 0 || ldc < n)
    return kq_fail(KQ_ERR_INVALID,
                   "%s: need k %% 128 == 0, lda >= k, lda %% 16 == 0, ldc >= n "
                   "(m=%lld n=%lld k=%lld lda=%lld ldc=%lld)",
                   fn, (long long)m, (long long)n, (long long)k, (long long)lda, (long long)ldc);
  if (m > INT32_MAX / 2 || n > INT32_MAX / 2 || k > INT32_MAX / 2 || (uint64_t)k * lin::BN > dma::MAX_RANGE ||
      (uint64_t)lda * lin::BM > dma::MAX_RANGE || (uint64_t)(m > n ? m : n) * (uint64_t)(k / 32) > dma::MAX_RANGE)
    return kq_fail(KQ_ERR_LIMIT, "%s: dimension too large", fn);
  return KQ_OK;
}

extern "C" int64_t kq_mx_linear_mx_workspace_size(int64_t m, int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k <= 0) return -1;
  return a8_scale_plane_bytes(m, k) + a8_scale_plane_bytes(n, k);
}

extern "C" int kq_mx_linear_mx(int a_fmt, const void* a_q, const uint8_t* a_scale, int64_t lda, int w_fmt,
                               const void* w_q, const uint8_t* w_scale, int64_t m, int64_t n, int64_t k,
                               int out_dtype, void* c, int64_t ldc, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  const char* fn = "kq_mx_linear_mx";
  if (int rc = check_linear_mx(fn, a_fmt, w_fmt, lda, m, n, k, out_dtype, ldc)) return rc;
  if (m == 0 || n == 0) return KQ_OK;
  if (!a_q || !a_scale || !w_q || !w_scale || !c) return kq_fail(KQ_ERR_INVALID, "%s: null buffer", fn);
  if (kq_misaligned(a_q, 16) || kq_misaligned(w_q, 16) || kq_misaligned(a_scale, 4) || kq_misaligned(w_scale, 4))
    return kq_fail(KQ_ERR_INVALID, "%s: a_q and w_q must be 16-byte aligned, the scales 4-byte aligned", fn);
  const int64_t need = kq_mx_linear_mx_workspace_size(m, n, k);
  if (!workspace || workspace_bytes < need || kq_misaligned(workspace, 256))
    return kq_fail(KQ_ERR_INVALID, "%s: workspace needs %lld bytes (256-byte aligned)", fn, (long long)need);
  hipStream_t st = (hipStream_t)stream;
  const uint8_t* ap = (const uint8_t*)a_q;
  const uint8_t* wp = (const uint8_t*)w_q;
  const hipError_t e =
      out_dtype == KQ_DT_BF16
          ? launch_linear_a8<0>(ap, a_scale, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, workspace, st)
          : launch_linear_a8<2>(ap, a_scale, lda, wp, w_scale, c, ldc, (int)m, (int)n, (int)k, workspace, st);
  return kq_check_launch(e, fn);
}

// kq_mx_linear_mm workspace: the input rows quantized, E4M3 [m, k] at 0 and
// E8M0 [m, k / 32] at the next 256-byte boundary, then kq_mx_linear_mx's.
static int64_t mm_scale_offset(int64_t m, int64_t k) { return (m * k + 255) / 256 * 256; }
static int64_t mm_mx_offset(int64_t m, int64_t k) { return mm_scale_offset(m, k) + a8_scale_plane_bytes(m, k); }

extern "C" int64_t kq_mx_linear_mm_workspace_size(int64_t m, int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k <= 0) return -1;
  return mm_mx_offset(m, k) + kq_mx_linear_mx_workspace_size(m, n, k);
}

extern "C" int kq_mx_linear_mm(int w_fmt, const void* a, int a_dtype, int64_t lda, const void* w_q,
                               const uint8_t* w_scale, int64_t m, int64_t n, int64_t k, int out_dtype, void* c,
                               int64_t ldc, void* workspace, int64_t workspace_bytes, void* stream) {
  const char* fn = "kq_mx_linear_mm";
  if (a_dtype != KQ_DT_BF16 && a_dtype != KQ_DT_F16 && a_dtype != KQ_DT_F32)
    return kq_fail(KQ_ERR_INVALID, "%s: input dtype must be bf16, f16 or f32", fn);
  if (lda < k) return kq_fail(KQ_ERR_INVALID, "%s: lda < k", fn);
  if (int rc = check_linear_mx(fn, KQ_FMT_MXFP8_E4M3, w_fmt, k, m, n, k, out_dtype, ldc)) return rc;
  if (m == 0 || n == 0) return KQ_OK;
  const int64_t need = kq_mx_linear_mm_workspace_size(m, n, k);
  if (!workspace || workspace_bytes < need || kq_misaligned(workspace, 256))
    return kq_fail(KQ_ERR_INVALID, "%s: workspace needs %lld bytes (256-byte aligned)", fn, (long long)need);
  uint8_t* xq = static_cast<uint8_t*>(workspace);
  uint8_t* xs = xq + mm_scale_offset(m, k);
  if (int rc = kq_mx_quantize(KQ_FMT_MXFP8_E4M3, a_dtype, a, lda, m, k, xq, xs, 0, stream)) return rc;
  return kq_mx_linear_mx(KQ_FMT_MXFP8_E4M3, xq, xs, k, w_fmt, w_q, w_scale, m, n, k, out_dtype, c, ldc,
                         xq + mm_mx_offset(m, k), need - mm_mx_offset(m, k), stream);
}
