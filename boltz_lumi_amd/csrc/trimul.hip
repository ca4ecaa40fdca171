// Fused triangle multiplication (outgoing / incoming) for gfx950.
//
// Replaces the reference's normalized_forward chain (multiplication.py:48-137:
// LN_in, p_in/g_in GEMMs, gate+mask+pack, torch.bmm, LN_out, p_out/g_out
// GEMMs, gate) with three kernels:
//
//  K1 trimul_proj     LN_in(x) -> [p_in; g_in] on MFMA -> a,b = bf16(p*sigmoid(g))*mask,
//                     written straight into the per-channel GEMM operand planes
//                     (k contiguous; the outgoing/incoming transpose is folded
//                     into which pair a block reads).
//  K2 trimul_contract O_c = A_c * B_c^T for the 128 channels, bf16 MFMA with fp32
//                     accumulation, LDS double buffering, XCD-grouped channels.
//  K3 trimul_out      LN_out(O) -> p_out, LN_in(x) -> g_out (recomputed instead of
//                     stored), y = p_out(.) * sigmoid(g_out(.)), then write y or
//                     add it into the fp32 residual stream in place.
//
// Operand planes (workspace, bf16, np = round_up(n, 128)):
//   A[c][r][t], B[c][r][t]   outgoing: A=a[r,t], B=b[r,t]; incoming: A=a[t,r], B=b[t,r]
//   O[c][i][j] = sum_t A[c][i][t] * B[c][j][t]
// so outgoing O = sum_k a[i,k] b[j,k] and incoming O = sum_k a[k,i] b[k,j]
// (the reference's bmm operands, multiplication.py:105-116).  Padding columns
// t >= n are written as zeros, so K2 runs unguarded over np.
#include <mutex>

#include "bmx_common.h"

using namespace bmx;

namespace {

constexpr int kPlaneTile = 256;        // plane padding granularity (the contraction's 256 x 256 tiles)

// ------------------------------------------------------------------ K1
// Persistent and weight-stationary: each wave keeps its [p_in; g_in] rows for
// 32 channels of a and of b in VGPRs for the life of the block, and the next
// tile's input rows are prefetched into registers while the current tile is
// projected, so HBM reads overlap the MFMA work.
constexpr int kP1 = 64;                // pairs per K1 tile (one plane row segment)
constexpr int kStage1 = kP1 + 8;       // staged plane rows (bf16)

template <bool kOutgoing>
__global__ __launch_bounds__(256, 2) void trimul_proj_kernel(const float* __restrict__ x,
                                                             const float* __restrict__ mask,
                                                             const float* __restrict__ ln_w,
                                                             const float* __restrict__ ln_b, float eps,
                                                             const bf16* __restrict__ w_in, bf16* __restrict__ a_pl,
                                                             bf16* __restrict__ b_pl, int n, int np) {
  __shared__ __attribute__((aligned(16))) bf16 xt[kP1 * kLdsRow];
  __shared__ __attribute__((aligned(16))) bf16 stage[2 * kC * kStage1];
  __shared__ __attribute__((aligned(16))) float msk[kP1];  // the tile's mask values, 0 for padding
  const int l = lane_id(), w = threadIdx.x >> 6, c0 = 32 * w;
  const int hw = threadIdx.x >> 5, hl = threadIdx.x & 31;
  const LnAffine aff = ln_affine(ln_w, ln_b, hl);
  const int tiles_x = np / kP1, total = np * tiles_x;
  const int64_t plane = (int64_t)np * np;

  // Weight rows for this wave: p(a), g(a), p(b), g(b) of channels c0..c0+31.
  bf16x8 wf[4][8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row0 = (q & 1) * 2 * kC + (q >> 1) * kC + c0;
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) wf[q][ks] = frag(w_in, kC, row0, ks);
  }

  // Input row p of a tile is pair (rp, t0+p) (outgoing) or (t0+p, rp) (incoming).
  // The tile's mask values (pair nt*32 + l%32 for this lane) are fetched with
  // its rows: a mask load next to its use is sunk under the padding test and
  // gets a vmcnt(0) wait, which would also wait for the whole prefetch.
  f32x4 pre[kP1 / 8];
  float mpre[kP1 / 32];
  auto fetch = [&](int tile) {
    const int rp = tile / tiles_x, t0 = (tile % tiles_x) * kP1;
    const int rc = min(rp, n - 1);  // padding rows / columns re-read row n-1 and are zeroed after the LN
#pragma unroll
    for (int nt = 0; nt < kP1 / 32; ++nt) {  // first, so that a wait for them leaves the rows in flight
      const int tc = min(t0 + nt * 32 + (l & 31), n - 1);
      mpre[nt] = mask[kOutgoing ? (int64_t)rc * n + tc : (int64_t)tc * n + rc];
    }
#pragma unroll
    for (int u = 0; u < kP1 / 8; ++u) {
      const int tc = min(t0 + hw + 8 * u, n - 1);
      const int64_t pair = kOutgoing ? (int64_t)rc * n + tc : (int64_t)tc * n + rc;
      pre[u] = load4(x + pair * kC + 4 * hl);
    }
  };

  // Tile k's operand rows leave the stage for the planes in iteration k+1,
  // right after its LayerNorm and before the next prefetch: vmcnt counts
  // stores in issue order, so stores issued before a prefetch have a whole
  // MFMA phase to retire before the next wait for that prefetch.
  auto store_planes = [&](int tile) {
    const int rp = tile / tiles_x, t0 = (tile % tiles_x) * kP1;
    // 2 operands x 128 channels x 8 chunks of 8 positions
#pragma unroll
    for (int u = 0; u < 2 * kC * (kP1 / 8) / 256; ++u) {
      const int idx = threadIdx.x + 256 * u;
      const int half = idx / (kC * (kP1 / 8)), ch = (idx / (kP1 / 8)) % kC, chunk = idx % (kP1 / 8);
      const bf16x8 v = *(const bf16x8*)(stage + (half * kC + ch) * kStage1 + chunk * 8);
      bf16* dst = (half ? b_pl : a_pl) + ch * plane + (int64_t)rp * np + t0 + chunk * 8;
      *(bf16x8*)dst = v;
    }
  };

  int tile = blockIdx.x, prev = -1;
  if (tile < total) fetch(tile);
  for (; tile < total; tile += gridDim.x) {
    const int rp = tile / tiles_x, t0 = (tile % tiles_x) * kP1;
    bool keep[kP1 / 8];
#pragma unroll
    for (int u = 0; u < kP1 / 8; ++u) keep[u] = rp < n && t0 + hw + 8 * u < n;
    ln128_half_rows(pre, keep, aff, eps);
#pragma unroll
    for (int u = 0; u < kP1 / 8; ++u) {
      bf16x4 o = {(bf16)pre[u][0], (bf16)pre[u][1], (bf16)pre[u][2], (bf16)pre[u][3]};
      *(bf16x4*)(xt + (hw + 8 * u) * kLdsRow + 4 * hl) = o;
    }
    // rows / columns past n (plane padding) are written as zeros
    const float mt = (rp < n && t0 + l < n) ? mpre[l >> 5] : 0.f;
    if (w == 0) msk[l] = mt;
    if (prev >= 0) store_planes(prev);
    __syncthreads();  // xt written; the stage has been read
    if (tile + (int)gridDim.x < total) fetch(tile + gridDim.x);

    // D[pair][ch]: A = normalised pairs, B = weight rows; lane l holds channel
    // c0 + l%32, and its registers 4q..4q+3 hold 4 consecutive pairs, which
    // leave as one 8-byte write into the channel's stage row.
#pragma unroll
    for (int nt = 0; nt < kP1 / 32; ++nt) {
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        f32x16 ap = zero16(), ag = zero16();
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          bf16x8 xf = frag(xt, kLdsRow, nt * 32, ks);
          ap = mfma32(xf, wf[2 * half][ks], ap);
          ag = mfma32(xf, wf[2 * half + 1][ks], ag);
        }
        bf16* srow = stage + (half * kC + c0 + (l & 31)) * kStage1;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int p0 = nt * 32 + drow(4 * q, l);
          const f32x4 m = *(const f32x4*)(msk + p0);
          // p * sigmoid(g) * mask, rounded once to the bf16 operand
          bf16x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = (bf16)(ap[4 * q + i] * sigmoid_f(ag[4 * q + i]) * m[i]);
          *(bf16x4*)(srow + p0) = o;
        }
      }
    }
    __syncthreads();  // stage written; xt has been read
    prev = tile;
  }
  if (prev >= 0) store_planes(prev);
}

// ------------------------------------------------------------------ K2
// Batched NT GEMM over channels: O_c[m][n] = sum_k A_c[m][k] * B_c[n][k].
// Operand tiles are copied global -> LDS by the DMA path (global_load_lds,
// 1 KB per wave instruction, lane l to byte 16 l), so the LDS tiles are dense
// rows of BK bf16 whose 16-byte chunks are XOR-swizzled by row: the fragment
// reads of 16 consecutive rows hit 16 distinct 4-bank groups.  NS stage
// buffers form a ring; the DMA of stage k + NS - 1 is issued while stage k is
// multiplied, so HBM / L2 latency is covered by NS - 1 stages of MFMA work
// and no staging registers are needed.  The MFMA computes D[n][m] (B as the
// A operand), so a lane holds 4 consecutive n of one row m: the result goes
// through LDS with 8-byte writes and leaves as 16-byte row stores.
// The DMA reads M0, which the compiler writes with an SALU instruction right
// before the asm; gfx9 needs one wait state between the two (s_nop 0), which
// the compiler's hazard recognizer inserts for its own LDS DMA but cannot see
// inside inline asm: without it the DMA may use the previous M0 and write its
// 1 KB over another stage region.
__device__ __forceinline__ void lds_dma16(const void* src, unsigned lds_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_addr) : "memory");
}

// s_waitcnt vmcnt(n) with the other counters left open (n < 64: the count's
// low 4 bits in [3:0], its high 2 bits in [15:14]).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt immediate");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// Persistent: block b takes the tiles b, b + G, b + 2G, ... (G = gridDim.x, a
// multiple of 8; tile T is what block T of a one-tile-per-block grid would
// do).  Blocks are dispatched round-robin over the 8 XCDs, so every block
// stays on one XCD, and tile T gives XCD T % 8 whole channels: a channel's
// operand planes stay in that XCD's L2.  Two stage buffers of BK-deep A / B
// tiles are filled by LDS DMA, one stage ahead.  After a tile's last stage
// the next tile's first stage goes to buffer 0 while the output is staged
// through the LDS past buffer 0 in two halves of BM / 2 rows; the next tile's
// first wait then leaves the epilogue's stores in flight (vmcnt counts stores
// too), so they drain under its stages.
template <int BM, int BN, int BK, int WM, int WN, int NS>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void trimul_contract_kernel(
    const bf16* __restrict__ A, const bf16* __restrict__ B, bf16* __restrict__ O, int np, int tiles_n,
    int tiles_per_ch, int tiles) {
  static_assert(NS == 2, "two stage buffers");
  constexpr int kWavesN = BN / WN;
  constexpr int kWaves = (BM / WM) * kWavesN;
  constexpr int kMi = WM / 32, kNi = WN / 32;
  constexpr int kCpr = BK / 8;                    // 16-byte chunks per tile row
  constexpr int kRpi = 1024 / (BK * 2);           // tile rows per DMA instruction
  constexpr int kSwz = 16 / kCpr;                 // rows per swizzle step
  static_assert(BK == 32 || BK == 64, "tile rows of 4 or 8 chunks");
  constexpr int kTileA = BM * BK * 2, kTileB = BN * BK * 2, kStage = kTileA + kTileB;
  constexpr int kDmaA = kTileA / 1024 / kWaves, kDmaB = kTileB / 1024 / kWaves;  // wave instructions per stage
  constexpr int kDma = kDmaA + kDmaB;
  static_assert(kDmaA * kWaves * 1024 == kTileA && kDmaB * kWaves * 1024 == kTileB, "tile/wave mismatch");
  constexpr int kORow = BN * 2 + 16;              // output staging row (bytes)
  constexpr int kHalf = BM / 2;                   // output rows staged at a time
  constexpr int kChunksRow = BN * 2 / 16;
  constexpr int kThreads = kWaves * 64;
  constexpr int kStoresHalf = kHalf * kChunksRow / kThreads;  // 16-byte stores per thread and half
  static_assert(kStoresHalf * kThreads == kHalf * kChunksRow && 2 * kStoresHalf < 64, "uniform epilogue stores");
  static_assert((BM / WM) % 2 == 0, "each half of the rows belongs to whole waves");
  constexpr int kStageOut = kStage;               // output staging: right after stage buffer 0
  constexpr int kSmem = NS * kStage > kStageOut + kHalf * kORow ? NS * kStage : kStageOut + kHalf * kORow;
  __shared__ __attribute__((aligned(16))) char smem[kSmem];

  const int64_t plane = (int64_t)np * np;
  const int t = threadIdx.x, l = lane_id(), wv = t >> 6;
  const int wm0 = (wv / kWavesN) * WM, wn0 = (wv % kWavesN) * WN;
  const unsigned lds0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)smem;
  auto operands = [&](int T, const bf16*& Ac, const bf16*& Bc, bf16*& Oc) {
    const int xcd = T & 7, idx = T >> 3;
    const int c = xcd + 8 * (idx / tiles_per_ch);
    const int tile = idx % tiles_per_ch;
    const int tm = tile / tiles_n, tn = tile % tiles_n;
    Ac = A + c * plane + (int64_t)tm * BM * np;
    Bc = B + c * plane + (int64_t)tn * BN * np;
    Oc = O + c * plane + (int64_t)(tm * BM) * np + tn * BN;
  };

  // DMA instruction u of this wave copies tile rows kRpi q .. kRpi q + kRpi - 1
  // (q = wave + kWaves u): lane l -> row kRpi q + l / kCpr, stored chunk
  // l % kCpr holding k-chunk (l % kCpr) ^ ((row / kSwz) % kCpr).
  auto dma_stage = [&](const bf16* Ac, const bf16* Bc, int k0, int buf) {
    const unsigned base = lds0 + buf * kStage;
#pragma unroll
    for (int u = 0; u < kDma; ++u) {
      const bool is_a = u < kDmaA;
      const int q = wv + kWaves * (is_a ? u : u - kDmaA);
      const int row = kRpi * q + l / kCpr, chunk = (l % kCpr) ^ ((row / kSwz) % kCpr);
      const bf16* src = (is_a ? Ac : Bc) + (int64_t)row * np + k0 + 8 * chunk;
      lds_dma16(src, __builtin_amdgcn_readfirstlane(base + (is_a ? 0 : kTileA) + 1024 * q));
    }
  };
  // Fragment (row0 + l % 32, k-step ks) of a tile at byte offset tile_off.
  auto sfrag = [&](const char* sb, int tile_off, int row0, int ks) -> bf16x8 {
    const int row = row0 + (l & 31), chunk = 2 * ks + (l >> 5);
    return *(const bf16x8*)(sb + tile_off + row * (BK * 2) + ((chunk ^ ((row / kSwz) % kCpr)) * 16));
  };

  const int kt_count = np / BK;  // >= 1: np is a multiple of 256
  const int G = gridDim.x;
  int T = blockIdx.x;
  bool prefetched = false;  // this tile's first stage is in buffer 0, requested before the last epilogue's stores
  while (T < tiles) {  // uniform over the block
    const bf16 *Ac, *Bc;
    bf16* Oc;
    operands(T, Ac, Bc, Oc);
    f32x16 acc[kMi][kNi];
#pragma unroll
    for (int i = 0; i < kMi; ++i)
#pragma unroll
      for (int j = 0; j < kNi; ++j) acc[i][j] = zero16();

    if (!prefetched) dma_stage(Ac, Bc, 0, 0);
    for (int kt = 0; kt < kt_count; ++kt) {
      // Stage kt is this wave's oldest outstanding memory operation except
      // for the previous epilogue's stores (first stage of a prefetched
      // tile); the barrier publishes every wave's copy and frees buffer
      // (kt + 1) % 2, read in stage kt - 1.
      if (kt == 0 && prefetched) wait_vm<2 * kStoresHalf>();
      else wait_vm<0>();
      __syncthreads();
      if (kt + 1 < kt_count) dma_stage(Ac, Bc, (kt + 1) * BK, (kt + 1) & 1);
      const char* sb = smem + (kt & 1) * kStage;
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8 af[kMi], bfr[kNi];
#pragma unroll
        for (int i = 0; i < kMi; ++i) af[i] = sfrag(sb, 0, wm0 + 32 * i, ks);
#pragma unroll
        for (int j = 0; j < kNi; ++j) bfr[j] = sfrag(sb, kTileA, wn0 + 32 * j, ks);
#pragma unroll
        for (int i = 0; i < kMi; ++i)
#pragma unroll
          for (int j = 0; j < kNi; ++j) acc[i][j] = mfma32(bfr[j], af[i], acc[i][j]);
      }
    }
    __syncthreads();  // every wave is done with the stage buffers

    int next = T + G;
    prefetched = next < tiles;
    if (prefetched) {  // the next tile's first stage, into buffer 0, ahead of this tile's stores
      const bf16 *An, *Bn;
      bf16* On;
      operands(next, An, Bn, On);
      dma_stage(An, Bn, 0, 0);
    }
    // acc[i][j] = D[n][m]: lane -> m = wm0 + 32 i + l%32, registers 4q'..4q'+3 ->
    // n = wn0 + 32 j + 8q' + 4(l/32) + 0..3, written as one 8-byte LDS store.
    // Rows [h kHalf, (h + 1) kHalf) belong to the waves with wm0 in that range.
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      if (wm0 / kHalf == h) {  // wave-uniform
#pragma unroll
        for (int i = 0; i < kMi; ++i)
#pragma unroll
          for (int j = 0; j < kNi; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int m = wm0 - h * kHalf + 32 * i + (l & 31), nn = wn0 + 32 * j + 8 * q + 4 * (l >> 5);
              const bf16x4 v = {(bf16)acc[i][j][4 * q], (bf16)acc[i][j][4 * q + 1], (bf16)acc[i][j][4 * q + 2],
                                (bf16)acc[i][j][4 * q + 3]};
              *(bf16x4*)(smem + kStageOut + m * kORow + nn * 2) = v;
            }
      }
      __syncthreads();
#pragma unroll
      for (int e0 = 0; e0 < kStoresHalf; ++e0) {
        const int e = t + kThreads * e0;
        const int m = e / kChunksRow, ch = e % kChunksRow;
        *(bf16x8*)(Oc + (int64_t)(h * kHalf + m) * np + 8 * ch) = *(const bf16x8*)(smem + kStageOut + m * kORow + 16 * ch);
      }
      __syncthreads();  // the staging rows are free again (and, after the second half, stage buffer 1)
    }
    T = next;
  }
}

// ------------------------------------------------------------------ K3
// Persistent and weight-stationary like K1.  A tile is 64 pairs (i, j0..j0+63).
// The input rows stay in registers (row layout: a half-wave per row, 4
// channels per lane) from the prefetch to the residual add, so x is read
// from HBM exactly once; the MFMA result is re-laid out through LDS (ybuf),
// where the residual is added.  Tile k's rows are stored from ybuf in
// iteration k+1, before the next prefetch is issued: vmcnt counts stores in
// issue order, so the wait for that prefetch does not wait for fresh stores.
// kScaled: the module output of frame row i is multiplied by row_scale[i]
// before it is written or added (PairformerLayer's row dropout mask).
constexpr int kP3 = 64;

template <bool kScaled>
__global__ __launch_bounds__(256, 2) void trimul_out_kernel(const float* x, const bf16* __restrict__ o_pl,
                                                            const float* __restrict__ in_w,
                                                            const float* __restrict__ in_b, float eps_in,
                                                            const float* __restrict__ out_w,
                                                            const float* __restrict__ out_b, float eps_out,
                                                            const bf16* __restrict__ w_pout,
                                                            const bf16* __restrict__ w_gout, void* out, int out_mode,
                                                            const float* __restrict__ row_scale, int n, int np) {
  // xo: LN_out(O) and xg: LN_in(x), pairs x channels; ybuf: the tile's fp32 output rows.
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kP3 * kLdsRow];
  __shared__ __attribute__((aligned(16))) float ybuf[kP3 * kYRow];
  bf16* xo = smem;
  bf16* xg = smem + kP3 * kLdsRow;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6, c0 = 32 * w;
  const int hw = t >> 5, hl = t & 31;
  const LnAffine aff_in = ln_affine(in_w, in_b, hl), aff_out = ln_affine(out_w, out_b, hl);
  const int tiles_x = (n + kP3 - 1) / kP3, total = n * tiles_x;
  const int64_t plane = (int64_t)np * np;
  const bool x_in_regs = out_mode == kOutResidual || (const void*)x == out;

  bf16x8 wp[8], wg[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    wp[ks] = frag(w_pout, kC, c0, ks);
    wg[ks] = frag(w_gout, kC, c0, ks);
  }

  constexpr int kRowsPer = kP3 / 8;                  // rows per half-wave
  constexpr int kOChunks = kC * (kP3 / 8) / 256;     // 16-byte product chunks per thread
  static_assert(kOChunks == 2 * (kP3 / 32), "one chunk per (pair block, k step)");
  // ident[ks]: B operand I[k][n] = (16 ks + k == n) for the transposing MFMA;
  // lane (half h, column n) holds k = 8h .. 8h+7.
  bf16x8 ident[2] = {};
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const int e = (l & 31) - 16 * ks - 8 * (l >> 5);
    if (e >= 0 && e < 8) ident[ks][e] = (bf16)1.f;
  }
  f32x4 px[kRowsPer];
  bf16x8 po[kOChunks];
  float prs = 1.f;
  auto fetch = [&](int tile) {
    const int i = tile / tiles_x, j0 = (tile % tiles_x) * kP3;
    if constexpr (kScaled) prs = row_scale[i];
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      const int j = j0 + hw + 8 * u;
      px[u] = j < n ? load4(x + ((int64_t)i * n + j) * kC + 4 * hl) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    // A operands of the transposing MFMA: pair block pb (32 pairs), k step ks
    // (16 pairs): channel c0 + l%32, pairs 32 pb + 16 ks + 8 (l/32) .. +7.
#pragma unroll
    for (int u = 0; u < kOChunks; ++u) {
      const int pb = u >> 1, ks = u & 1;
      po[u] = *(const bf16x8*)(o_pl + (c0 + (l & 31)) * plane + (int64_t)i * np + j0 + 32 * pb + 16 * ks +
                               8 * (l >> 5));
    }
  };

  // Rows of ybuf (residual already added where it is held in registers) to
  // the output; thread (half-wave row, 4 channels) as in the residual add.
  auto store_rows = [&](int tile) {
    const int i = tile / tiles_x, j0 = (tile % tiles_x) * kP3;
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      const int p = hw + 8 * u, j = j0 + p;
      if (j < n) {
        const f32x4 y = *(const f32x4*)(ybuf + p * kYRow + 4 * hl);
        const int64_t off = ((int64_t)i * n + j) * kC + 4 * hl;
        if (out_mode == kOutBF16 || (out_mode == kOutAccumulate && !x_in_regs))
          store_row4(out, off, y, y, out_mode, false);
        else
          *(f32x4*)((float*)out + off) = y;
      }
    }
  };

  int tile = blockIdx.x, prev = -1;
  if (tile < total) fetch(tile);
  for (; tile < total; tile += gridDim.x) {
    const float rs = prs;
    f32x4 xc[kRowsPer];
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      xc[u] = px[u];
      f32x4 y = ln128_half(px[u], aff_in, eps_in);
      bf16x4 o = {(bf16)y[0], (bf16)y[1], (bf16)y[2], (bf16)y[3]};
      *(bf16x4*)(xg + (hw + 8 * u) * kLdsRow + 4 * hl) = o;
    }
    // Transpose O (channel-major planes) into xo[pair][channel] with an
    // identity B operand: D[ch][pair] = O[ch][k] * I[k][pair] puts 4
    // consecutive channels of one pair in each register group, written as
    // one 8-byte LDS store (a 2-byte scatter here costs 4-8-way bank conflicts).
#pragma unroll
    for (int pb = 0; pb < kP3 / 32; ++pb) {
      f32x16 d = mfma32(po[2 * pb], ident[0], zero16());
      d = mfma32(po[2 * pb + 1], ident[1], d);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16x4 v = {(bf16)d[4 * q], (bf16)d[4 * q + 1], (bf16)d[4 * q + 2], (bf16)d[4 * q + 3]};
        *(bf16x4*)(xo + (32 * pb + (l & 31)) * kLdsRow + c0 + 8 * q + 4 * (l >> 5)) = v;
      }
    }
    if (prev >= 0) store_rows(prev);
    __syncthreads();
    if (tile + (int)gridDim.x < total) fetch(tile + gridDim.x);
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      bf16* row = xo + (hw + 8 * u) * kLdsRow + 4 * hl;
      f32x4 v = {(float)row[0], (float)row[1], (float)row[2], (float)row[3]};
      f32x4 y = ln128_half(v, aff_out, eps_out);
      bf16x4 o = {(bf16)y[0], (bf16)y[1], (bf16)y[2], (bf16)y[3]};
      *(bf16x4*)row = o;
    }
    __syncthreads();

    // D[pair][ch]: A = normalised pairs, B = weight rows; lane l holds channel c0 + l%32.
    f32x16 res[kP3 / 32];
#pragma unroll
    for (int nt = 0; nt < kP3 / 32; ++nt) {
      f32x16 ay = zero16(), ag = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        ay = mfma32(frag(xo, kLdsRow, nt * 32, ks), wp[ks], ay);
        ag = mfma32(frag(xg, kLdsRow, nt * 32, ks), wg[ks], ag);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        res[nt][r] = rbf(ay[r] * sigmoid_f(ag[r]));  // the bf16 module output
        if constexpr (kScaled) res[nt][r] *= rs;
      }
    }
#pragma unroll
    for (int nt = 0; nt < kP3 / 32; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) ybuf[(nt * 32 + drow(r, l)) * kYRow + c0 + (l & 31)] = res[nt][r];
    __syncthreads();
    if (out_mode == kOutResidual || (out_mode == kOutAccumulate && x_in_regs)) {
#pragma unroll
      for (int u = 0; u < kRowsPer; ++u) {
        f32x4* row = (f32x4*)(ybuf + (hw + 8 * u) * kYRow + 4 * hl);
        *row = xc[u] + *row;
      }
    }
    prev = tile;
  }
  if (prev >= 0) store_rows(prev);
}

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// The three kernels of one module on `workspace` (3 planes of 128 x np x np bf16).
int launch(const float* x, const float* mask, int ni, int outgoing, const float* norm_in_w, const float* norm_in_b,
           float eps_in, const bf16* w_in, const float* norm_out_w, const float* norm_out_b, float eps_out,
           const bf16* w_pout, const bf16* w_gout, void* out, int out_mode, const float* row_scale, void* workspace,
           int stages, hipStream_t stream) {
  const int np = (int)round_up(ni, kPlaneTile);
  const int64_t plane = (int64_t)np * np * kC;
  bf16* a_pl = (bf16*)workspace;
  bf16* b_pl = a_pl + plane;
  bf16* o_pl = b_pl + plane;

  if (stages & 1) {
    const int total = np * (np / kP1);
    const int grid = total < 2 * device_cu_count() ? total : 2 * device_cu_count();
    if (outgoing)
      trimul_proj_kernel<true><<<dim3(grid), 256, 0, stream>>>(x, mask, norm_in_w, norm_in_b, eps_in, w_in, a_pl, b_pl,
                                                               ni, np);
    else
      trimul_proj_kernel<false><<<dim3(grid), 256, 0, stream>>>(x, mask, norm_in_w, norm_in_b, eps_in, w_in, a_pl,
                                                                b_pl, ni, np);
    if (int rc = check_launch("trimul_proj")) return rc;
  }
  if (stages & 2) {
    // Two 64-deep stages: 32-deep stages in a 3- or 4-stage ring measured
    // slower (more barriers per k), as did register staging of the operands.
    constexpr int BM = 256, BN = 256, BK = 64, WM = 64, WN = 128, NS = 2;
    const int tiles_n = np / BN, tiles_per_ch = (np / BM) * tiles_n;
    // persistent, one block per CU (its LDS holds two stages), a multiple of 8 so each block keeps one XCD
    const int tiles = kC * tiles_per_ch;
    const int grid = std::min(tiles, 8 * ((device_cu_count() + 7) / 8));
    trimul_contract_kernel<BM, BN, BK, WM, WN, NS>
        <<<dim3(grid), (BM / WM) * (BN / WN) * 64, 0, stream>>>(a_pl, b_pl, o_pl, np, tiles_n, tiles_per_ch, tiles);
    if (int rc = check_launch("trimul_contract")) return rc;
  }
  if (stages & 4) {
    const int total = ni * ((ni + kP3 - 1) / kP3);
    const int grid = total < 2 * device_cu_count() ? total : 2 * device_cu_count();
    if (row_scale)
      trimul_out_kernel<true><<<dim3(grid), 256, 0, stream>>>(x, o_pl, norm_in_w, norm_in_b, eps_in, norm_out_w,
                                                              norm_out_b, eps_out, w_pout, w_gout, out, out_mode,
                                                              row_scale, ni, np);
    else
      trimul_out_kernel<false><<<dim3(grid), 256, 0, stream>>>(x, o_pl, norm_in_w, norm_in_b, eps_in, norm_out_w,
                                                               norm_out_b, eps_out, w_pout, w_gout, out, out_mode,
                                                               nullptr, ni, np);
    if (int rc = check_launch("trimul_out")) return rc;
  }
  return BMX_OK;
}

// Checks shared by both entry points (everything but the workspace).
int check_args(const char* fn, const float* x, const float* mask, int64_t n, int64_t max_n, const float* norm_in_w,
               const float* norm_in_b, float eps_in, const void* w_in, const float* norm_out_w,
               const float* norm_out_b, float eps_out, const void* w_pout, const void* w_gout, const void* out,
               int out_mode) {
  BMX_REQUIRE(n >= 0 && n <= max_n, "%s: n must be in [0, %lld] (got %lld)", fn, (long long)max_n, (long long)n);
  BMX_REQUIRE(out_mode >= 0 && out_mode <= 3, "%s: out_mode must be 0 (bf16), 1 (fp32), 2 (fp32 +=) or 3 (fp32 x + y)",
              fn);
  BMX_REQUIRE(eps_in > 0.f && eps_out > 0.f, "%s: eps must be positive", fn);
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(x && mask && norm_in_w && norm_in_b && w_in && norm_out_w && norm_out_b && w_pout && w_gout && out,
              "%s: null pointer", fn);
  BMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)w_in % 16 == 0 && (uintptr_t)w_pout % 16 == 0 &&
                  (uintptr_t)w_gout % 16 == 0,
              "%s: x and weights must be 16-byte aligned", fn);
  return BMX_OK;
}

// ---------------------------------------------------------------------------
// Allocation-free variant.  Its operand planes live in `scratch`, a static
// device array that every GPU the library runs on holds for the life of the
// process.  Host code never passes `scratch` itself (in host code the name is
// a host-side stand-in, not a device address): the device address is looked
// up once per device with hipGetSymbolAddress, with that device current, and
// kept in g_scratch.
constexpr int kNoAllocMaxN = 256;
constexpr size_t kScratchBytes = (size_t)3 * kC * kNoAllocMaxN * kNoAllocMaxN * sizeof(bf16);  // 48 MiB
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) char scratch[kScratchBytes];

namespace {

// Device address of this device's `scratch` (looked up on the first call on
// the device), or nullptr with the error set.
void* scratch_address(int* rc) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    *rc = set_error(BMX_ELAUNCH, "bmx_trimul_fwd_noalloc: no usable current device (%s)", hipGetErrorString(e));
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr) {
      *rc = set_error(BMX_ELAUNCH, "bmx_trimul_fwd_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                      hipGetErrorString(e));
      return nullptr;
    }
    g_scratch[dev] = ptr;
  }
  return g_scratch[dev];
}

}  // namespace

extern "C" {

size_t bmx_trimul_workspace_bytes(int64_t n) {
  if (n <= 0) return 0;
  int64_t np = round_up(n, kPlaneTile);
  return (size_t)(3 * (int64_t)kC * np * np * (int64_t)sizeof(bf16));
}

int bmx_trimul_fwd(const float* x, const float* mask, int64_t n, int outgoing, const float* norm_in_w,
                   const float* norm_in_b, float eps_in, const void* w_in, const float* norm_out_w,
                   const float* norm_out_b, float eps_out, const void* w_pout, const void* w_gout, void* out,
                   int out_mode, const float* row_scale, void* workspace, size_t workspace_bytes, int stages,
                   hipStream_t stream) {
  const char* fn = "bmx_trimul_fwd";
  BMX_REQUIRE(stages >= 1 && stages <= 7, "bmx_trimul_fwd: stages must be a non-empty subset of 1|2|4");
  if (int rc = check_args(fn, x, mask, n, 16384, norm_in_w, norm_in_b, eps_in, w_in, norm_out_w, norm_out_b, eps_out,
                          w_pout, w_gout, out, out_mode))
    return rc;
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(workspace && workspace_bytes >= bmx_trimul_workspace_bytes(n),
              "bmx_trimul_fwd: workspace too small (%zu < %zu bytes)", workspace_bytes,
              bmx_trimul_workspace_bytes(n));
  BMX_REQUIRE((uintptr_t)workspace % 16 == 0, "bmx_trimul_fwd: workspace must be 16-byte aligned");
  return launch(x, mask, (int)n, outgoing, norm_in_w, norm_in_b, eps_in, (const bf16*)w_in, norm_out_w, norm_out_b,
                eps_out, (const bf16*)w_pout, (const bf16*)w_gout, out, out_mode, row_scale, workspace, stages,
                stream);
}

int bmx_trimul_fwd_noalloc(const float* x, const float* mask, int64_t n, int outgoing, const float* norm_in_w,
                           const float* norm_in_b, float eps_in, const void* w_in, const float* norm_out_w,
                           const float* norm_out_b, float eps_out, const void* w_pout, const void* w_gout, void* out,
                           int out_mode, hipStream_t stream) {
  const char* fn = "bmx_trimul_fwd_noalloc";
  if (int rc = check_args(fn, x, mask, n, kNoAllocMaxN, norm_in_w, norm_in_b, eps_in, w_in, norm_out_w, norm_out_b,
                          eps_out, w_pout, w_gout, out, out_mode))
    return rc;
  if (n == 0) return BMX_OK;
  int rc = BMX_OK;
  void* ws = scratch_address(&rc);
  if (ws == nullptr) return rc;
  // The projection writes every element of the A and B planes (padding as
  // zeros) and the contraction every element of O, so nothing left in the
  // scratch by an earlier call is read: no clearing is needed.
  return launch(x, mask, (int)n, outgoing, norm_in_w, norm_in_b, eps_in, (const bf16*)w_in, norm_out_w, norm_out_b,
                eps_out, (const bf16*)w_pout, (const bf16*)w_gout, out, out_mode, nullptr, ws, 7, stream);
}

}  // extern "C"
