// Fused triangle attention (starting / ending node) for gfx950.
//
// Replaces TriangleAttention.forward + the reference's ordered_triangle_forward
// (triangle.py:32-104, 107-146) and its fused softmax kernels
// (kernels/triangle_softmax.py, kernels/triangle_block_softmax_hip.cu).  The
// [I, H, Q, K] score tensor is never materialised.
//
// All kernels work in the "row frame" x'[i][j]: x'[i][j] = x[i][j] for the
// starting node and x[j][i] for the ending node (upstream transposes x and the
// mask, triangle.py:131), so only the x read and the output write differ.
//
//  K1 triattn_proj   LN(x') -> q (pre-scaled by log2(e)/sqrt(d)), k, v^T and the
//                    triangle bias tb[h][q][k] = log2(e) * linear(x')[q,k,h] on
//                    MFMA; mask bias mb[i][k] = log2(e) * inf * (mask'[i][k] - 1).
//  K2 triattn_core   one block per (2 rows i, head h, 128 queries); per 64-key
//                    stage S^T = K Q^T + tb^T (+ mb for masked rows) with the
//                    bias as the MFMA C operand, online softmax in base 2
//                    (fp32), O^T += V^T P^T with P kept in registers (bf16).
//  K3 triattn_out    o * sigmoid(linear_g(LN(x')) + b_g) -> linear_o + b_o, then
//                    write or add into the fp32 residual in place.
//
// Workspace (np = round_up(n, 128)):
//   q[i][h][j][d], k[i][h][j][d], vt[i][h][d][j']  bf16, i < np, j < np, where
//     j' = (j & ~31) + vperm(j & 31) permutes keys inside each 32-key block
//   tb: H x np x np bf16 in B-operand order (tb_offset; k >= n is kPadBias), mb[i][k] fp32,
//   o[i][j][h*32+d] bf16 (n x n)
#include "bmx_common.h"

using namespace bmx;

namespace {

constexpr int kH = 4, kD = 32, kPad = 256;  // row padding: a multiple of the projection and attention tiles
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kProjRows = 3 * kC + 32;  // q, k, v, then H triangle-bias rows (+ zero rows)
// Triangle-bias storage type: bf16, as upstream's bf16 path rounds the bias.
// The attention core adds it with an MFMA (identity A operand, bias as the B
// operand), so it needs no conversion to fp32.
using tb_t = bf16;
// Bias of padding keys (k >= n).  Finite, because the identity MFMA multiplies
// every bias entry by 0 for the other 15 keys of its tile (0 * -inf = NaN);
// exp2 of it is still exactly 0.
constexpr float kPadBias = -1e30f;

struct Layout {
  int n, np;
  bf16 *q, *k, *vt, *o;
  tb_t* tb;
  float* mb;
  // Per row i and 64-key tile: the first masked key of the tile (n if none;
  // -2 if some key's mask is neither 0 nor 1) and the last open key (-1 if
  // none), keys < n only; written by the projection, read by the attention
  // core to pick its path per block.
  int2* keyspan;
};

__host__ __device__ inline int64_t qkv_elems(int np) { return (int64_t)np * kH * np * kD; }

// V^T rows keep each 32-key block in the order in which the attention core's
// P operand holds keys: storage slot 8g + 4a + c holds key 16a + 4g + c, so the
// 8 keys of lane group g are one contiguous 16-byte read.
__host__ __device__ inline int vperm(int key_in_block) {
  return ((key_in_block >> 2) & 3) * 8 + ((key_in_block >> 4) & 1) * 4 + (key_in_block & 3);
}

// The triangle bias is stored in the attention core's B-operand order: for
// head h, query block qb (16 queries) and key block kb (16 keys), one 512-byte
// run holds, for lane L = 16 (k % 16 / 8) + q % 16 (L < 32), the 8 keys
// 16 kb + 8 (L / 16) + 0..7 of query 16 qb + L % 16, so a bias load of the
// core reads 32 lanes x 16 contiguous bytes.
// (32-bit: H * np * np < 2^31 for n <= 8192.)
__host__ __device__ inline int tb_offset(int np, int h, int q, int k) {
  const int nb = np / 16;
  return ((h * nb + q / 16) * nb + k / 16) * 256 + (((k & 15) >> 3) * 16 + (q & 15)) * 8 + (k & 7);
}

template <typename TIn>
__device__ __forceinline__ const TIn* xrow(const TIn* x, int n, int starting, int i, int j) {
  int64_t pair = starting ? (int64_t)i * n + j : (int64_t)j * n + i;
  return x + pair * kC;
}

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ------------------------------------------------------------------ K1
// Persistent and weight-stationary.  Wave w keeps head w's q, k and v weight
// rows (3 x 32 rows, 32x32x16 operands) and the 4 triangle-bias rows (16x16x32
// A operands) in VGPRs for the block's lifetime.  A tile is 64 positions
// (i, j0..j0+63) of the row frame over the padded np x np range, so padding
// rows and keys get their zero / -inf values from the same code; the next
// tile's input rows are prefetched into registers during the current tile's
// MFMAs.  q, k and v^T leave through an LDS stage in their HBM order and are
// stored in the next iteration, before the next prefetch: vmcnt counts
// stores in issue order, so a wait for the prefetch never waits for fresh
// stores.  q and k are computed as D[d][pair] and v^T as D[pair][d], so each
// lane holds 4 consecutive elements of one stage row (one 8-byte LDS write).
constexpr int kP1 = 64;
constexpr int kQRow = kD + 8;   // staged q / k row of one pair (bf16, 80 bytes)
constexpr int kVRow = kP1 + 8;  // staged v^T row of one head dim (bf16, 144 bytes)

template <typename TIn, bool starting>
__global__ __launch_bounds__(256, 2) void triattn_proj_kernel(const TIn* __restrict__ x, const float* __restrict__ mask,
                                                              const float* __restrict__ ln_w,
                                                              const float* __restrict__ ln_b, float eps,
                                                              const bf16* __restrict__ w_proj, float inf,
                                                              Layout L) {
  __shared__ __attribute__((aligned(16))) bf16 xt[kP1 * kLdsRow];
  __shared__ __attribute__((aligned(16))) bf16 sq[kH * kP1 * kQRow];
  __shared__ __attribute__((aligned(16))) bf16 sk[kH * kP1 * kQRow];
  __shared__ __attribute__((aligned(16))) bf16 sv[kH * kD * kVRow];
  const int n = L.n, np = L.np;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6, h = w, g = l >> 4, lq = l & 15;
  const int hw = t >> 5, hl = t & 31;
  const LnAffine aff = ln_affine(ln_w, ln_b, hl);
  const int tiles_x = np / kP1, total = np * tiles_x;
  const float qscale = kLog2e / sqrtf((float)kD);

  // Weight rows: q, k, v of head h are rows 32h, 128 + 32h, 256 + 32h; the
  // triangle-bias rows 384..387 (then zero rows) as A[l%16][32 ks + 8g ..].
  bf16x8 wq[8], wk[8], wv[8], wb[4];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    wq[ks] = frag(w_proj, kC, 32 * h, ks);
    wk[ks] = frag(w_proj, kC, kC + 32 * h, ks);
    wv[ks] = frag(w_proj, kC, 2 * kC + 32 * h, ks);
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) wb[ks] = *(const bf16x8*)(w_proj + (3 * kC + lq) * kC + 32 * ks + 8 * g);

  // Input rows and the mask value of position j0 + t % 64 (clamped into range:
  // every load is unconditional, padding rows are zeroed after the LayerNorm).
  constexpr int kRowsPer = kP1 / 8;
  f32x4 px[kRowsPer];
  float mpre = 1.f;
  auto fetch = [&](int tile) {
    const int i = min(tile / tiles_x, n - 1), j0 = (tile % tiles_x) * kP1;
    if (mask) {
      const int jc = min(j0 + (t & (kP1 - 1)), n - 1);
      mpre = starting ? mask[(int64_t)i * n + jc] : mask[(int64_t)jc * n + i];
    }
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) px[u] = load4(xrow(x, n, starting, i, min(j0 + hw + 8 * u, n - 1)) + 4 * hl);
  };

  // Stage -> HBM, 16-byte chunks: q and k are 4 KB runs per head, v^T 128-byte runs per (head, dim).
  auto store_stage = [&](int tile) {
    const int i = tile / tiles_x, j0 = (tile % tiles_x) * kP1;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = t + 256 * u, hh = c >> 8, p = (c >> 2) & (kP1 - 1), part = c & 3;
      const int64_t off = (((int64_t)i * kH + hh) * np + j0 + p) * kD + 8 * part;
      *(bf16x8*)(L.q + off) = *(const bf16x8*)(sq + (hh * kP1 + p) * kQRow + 8 * part);
      *(bf16x8*)(L.k + off) = *(const bf16x8*)(sk + (hh * kP1 + p) * kQRow + 8 * part);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = t + 256 * u, hh = c >> 8, d = (c >> 3) & (kD - 1), part = c & 7;
      *(bf16x8*)(L.vt + (((int64_t)i * kH + hh) * kD + d) * np + j0 + 8 * part) =
          *(const bf16x8*)(sv + (hh * kD + d) * kVRow + 8 * part);
    }
  };

  int tile = blockIdx.x, prev = -1;
  if (tile < total) fetch(tile);
  for (; tile < total; tile += gridDim.x) {
    const int i = tile / tiles_x, j0 = (tile % tiles_x) * kP1;
    bool keep[kRowsPer];
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) keep[u] = i < n && j0 + hw + 8 * u < n;
    ln128_half_rows(px, keep, aff, eps);  // px is fetched again after the barrier
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      const bf16x4 o = {(bf16)px[u][0], (bf16)px[u][1], (bf16)px[u][2], (bf16)px[u][3]};
      *(bf16x4*)(xt + (hw + 8 * u) * kLdsRow + 4 * hl) = o;
    }
    if (t < kP1) {
      // mask bias mb[i][j] = log2(e) * inf * (mask'[i][j] - 1); 0 outside n x n
      const int j = j0 + t;
      const bool valid = i < n && j < n;
      const float mbv = valid ? inf * (mpre - 1.f) * kLog2e : 0.f;
      L.mb[(int64_t)i * np + j] = mbv;
      // masked keys: closed (mask 0) by index, fractional ones as -2 (they pin the block to the masked path)
      int fm = valid && mbv != 0.f ? (mpre == 0.f ? j : -2) : n, lo = valid && mbv == 0.f ? j : -1;
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) {
        fm = min(fm, __shfl_xor(fm, d, kWave));
        lo = max(lo, __shfl_xor(lo, d, kWave));
      }
      if (t == 0) L.keyspan[(int64_t)i * (np / kP1) + j0 / kP1] = make_int2(fm, lo);
    }
    if (prev >= 0) store_stage(prev);
    __syncthreads();  // xt written; the stage has been read
    if (tile + (int)gridDim.x < total) fetch(tile + gridDim.x);

#pragma unroll
    for (int nt = 0; nt < kP1 / 32; ++nt) {
      bf16x8 xf[8];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) xf[ks] = frag(xt, kLdsRow, nt * 32, ks);
      // q, k: D[d][pair], lane -> pair nt*32 + l%32, registers 4q'..4q'+3 -> d 8q' + 4(l/32) + 0..3.
#pragma unroll
      for (int kind = 0; kind < 2; ++kind) {
        f32x16 acc = zero16();
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) acc = mfma32(kind == 0 ? wq[ks] : wk[ks], xf[ks], acc);
        bf16* dst = (kind == 0 ? sq : sk) + (h * kP1 + nt * 32 + (l & 31)) * kQRow + 4 * (l >> 5);
        const float sc = kind == 0 ? qscale : 1.f;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const bf16x4 v = {(bf16)(acc[4 * q4] * sc), (bf16)(acc[4 * q4 + 1] * sc), (bf16)(acc[4 * q4 + 2] * sc),
                            (bf16)(acc[4 * q4 + 3] * sc)};
          *(bf16x4*)(dst + 8 * q4) = v;
        }
      }
      // v^T: D[pair][d], lane -> d = l%32, registers 4q'..4q'+3 -> pairs nt*32 + 8q' + 4(l/32) + 0..3,
      // stored at their permuted key slots (vperm keeps runs of 4 keys together).
      f32x16 av = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) av = mfma32(xf[ks], wv[ks], av);
      bf16* vdst = sv + (h * kD + (l & 31)) * kVRow + nt * 32;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const bf16x4 v = {(bf16)av[4 * q4], (bf16)av[4 * q4 + 1], (bf16)av[4 * q4 + 2], (bf16)av[4 * q4 + 3]};
        *(bf16x4*)(vdst + vperm(8 * q4 + 4 * (l >> 5))) = v;
      }
    }
    {
      // Triangle bias for pairs j0 + 16w .. +15: D[head][pair] on 16x16x32,
      // lanes of group 0 hold heads 0..3 in registers 0..3.
      f32x4 ab = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        ab = mfma16(wb[ks], *(const bf16x8*)(xt + (16 * w + lq) * kLdsRow + 32 * ks + 8 * g), ab);
      const int j = j0 + 16 * w + lq;
      if (g == 0) {
        tb_t* dst = L.tb + tb_offset(np, 0, i, j);
        const int head_stride = np * np;  // tb_offset(np, h + 1, ..) - tb_offset(np, h, ..)
#pragma unroll
        for (int r = 0; r < kH; ++r) dst[r * head_stride] = (tb_t)(j < n ? ab[r] * kLog2e : kPadBias);
      }
    }
    __syncthreads();  // the stage is written; xt has been read
    prev = tile;
  }
  if (prev >= 0) store_stage(prev);
}

// ------------------------------------------------------------------ K2
// MFMA shape of the attention core: v_mfma_f32_16x16x32_bf16 (lane l, group
// g = l / 16): A holds A[l%16][8g .. 8g+7], B holds B[8g .. 8g+7][l%16], D
// register r holds D[4g + r][l%16].  With 16 queries per wave the head dim
// (32) is one K step and a wave's per-row state is small, so 8 waves x 2 rows
// fit at 4 waves per SIMD.
constexpr int kKT = 64;  // keys per pipeline stage

// Stage buffers are filled by LDS DMA (global_load_lds_dwordx4: one wave
// instruction copies 1 KB, lane l to byte 16 l), so the K and V^T tiles are
// dense and XOR-swizzled in 16-byte chunks instead of padded; the MFMA operand
// reads of 16 consecutive lanes then hit 16 distinct 4-bank groups:
//   K tile   (64 keys x 32 d)  key k, d chunk c (8 dims)  -> chunk 4k + (c ^ ((k >> 2) & 3))
//   V^T tile (32 d x 64 keys)  dim d, key chunk c (8 keys) -> chunk 8d + (c ^ ((d >> 1) & 7))
constexpr int kTileBytes = kKT * kD * 2;  // one K or V^T tile of one row

// Rescale the running output only when a query's max grows by more than
// 2^kLazy: until then p = exp2(s - m) stays <= 2^kLazy, exact in fp32/bf16.
constexpr float kLazy = 8.f;

constexpr int kCoreWaves = 8;              // waves per attention block
constexpr int kCoreQ = 16 * kCoreWaves;    // queries per attention block
constexpr int kCoreThreads = 64 * kCoreWaves;

// Rows i processed together by one block: every triangle-bias tile loaded
// into registers serves all of them, which divides the bias traffic
// (N x the [H, N, N] bias per direction) by kRows.
constexpr int kRows = 2;

// Blocks are dispatched round-robin over the 8 XCDs.  A "column" is one
// (head, query tile); every XCD owns a contiguous run of columns, so the
// triangle-bias rows those columns re-read for every row group stay in that
// XCD's L2 instead of being fetched again from HBM / MALL.
__host__ __device__ inline int core_qtiles(int n) { return (n + kCoreQ - 1) / kCoreQ; }
__host__ __device__ inline int core_cols_per_xcd(int n) { return (kH * core_qtiles(n) + 7) / 8; }
__host__ __device__ inline int core_row_groups(int n) { return (n + kRows - 1) / kRows; }

// LDS stage buffer, per block: K and V^T tiles of the kRows rows, every wave's
// triangle-bias B tiles for the stage (4 tiles x 512 B), and the rows' mask
// bias (masked blocks only).
constexpr int kBiasWaveBytes = 4 * 512;
constexpr int kOffK = 0, kOffV = kRows * kTileBytes, kOffBias = 2 * kRows * kTileBytes;
constexpr int kOffMb = kOffBias + kCoreWaves * kBiasWaveBytes;
constexpr int kStageBytes = kOffMb + kRows * kKT * 4;

// One LDS DMA: 64 lanes x 16 bytes from per-lane global addresses to
// lds_addr + 16 * lane.  Issued as inline asm so that the compiler does not
// wait for it before unrelated LDS reads: the kernel waits for its DMAs
// explicitly (s_waitcnt vmcnt) before the barrier that publishes them.
// The DMA reads M0, which the compiler writes with an SALU instruction right
// before the asm; gfx9 needs one wait state between the two (s_nop 0), which
// the compiler's hazard recognizer inserts for its own LDS DMA but cannot see
// inside inline asm: without it the DMA may use the previous M0 and write its
// 1 KB over another stage region.
__device__ __forceinline__ void lds_dma16(const void* src, unsigned lds_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_addr) : "memory");
}
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
__device__ __forceinline__ float max3f(float a, float b, float c) { return fmaxf(fmaxf(a, b), c); }

// SPEC (unmasked rows only): after the first stage the offset m is frozen and
// the running max is not computed; p = exp2(s - m) may then exceed 2^kLazy.
// The offset is also shared by the block's rows (the max of their first-stage
// maxima), so the bias tile minus m, which does not depend on the row, is
// formed by one identity MFMA per key tile and is the C operand of every
// row's K Q^T.  That is exact up to a common scale as long as nothing
// overflows and no row's sum falls towards the fp32 underflow range, which the
// end of the pass checks (every row sum in [2^-60, 2^100], every output
// finite); otherwise nothing is written and false is returned, and the caller
// redoes the block with per-row tracked maxima.
//
// KEYMASK (speculative pass for key-padded rows): every row of the block has
// at least one unmasked key and its masked keys form a suffix of the key
// range (token padding gives exactly this: pair (i, k) is masked for the
// padded tokens k).  Stages from `mask_k0` on add the rows' mask bias to the
// C operand as the masked path does, so masked keys contribute exp2 of about
// -1.4e9, i.e. exactly 0; keys from `kend` on are masked for every row and
// are skipped.  The result is the masked path's up to the offset.
template <bool MASKED, bool SPEC, bool KEYMASK = false>
__device__ __forceinline__ bool core_rows(const Layout& L, int i0, int h, int q0, char* lds, int kend, int mask_k0) {
  static_assert(!(MASKED && SPEC), "speculation is for unmasked rows");
  static_assert(!KEYMASK || SPEC, "key-padded rows use the speculative pass");
  constexpr int G = kRows;
  const int n = L.n, np = L.np;
  // w is wave-uniform: read into an SGPR so that the DMA job set-up and the
  // LDS (M0) addresses below stay scalar.
  const int l = lane_id(), g = l >> 4, lq = l & 15, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nk = kend;  // a multiple of kKT, at most round_up(n, kKT)
  const unsigned lds0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds;
  const bf16* kb[G];
  const bf16* vb[G];
  bf16x8 qf[G];
#pragma unroll
  for (int r = 0; r < G; ++r) {
    const int i = min(i0 + r, n - 1);  // rows past n repeat row n-1 and are not stored
    kb[r] = L.k + ((int64_t)i * kH + h) * np * kD;
    vb[r] = L.vt + ((int64_t)i * kH + h) * kD * np;
    // Q^T (B operand): query q0 + l%16, head dims 8g .. 8g+7
    qf[r] = *(const bf16x8*)(L.q + (((int64_t)i * kH + h) * np + q0 + lq) * kD + 8 * g);
  }

  // DMA jobs of one stage.  K / V^T: 4 quarters per (row, kind), job
  // 8 r + 4 kind + quarter, wave w takes jobs w and w + 8.  Bias: every wave
  // copies its own 16 queries' 4 tiles (2 KB, contiguous in the bias layout).
  // Mask bias: wave 0's first 32 lanes copy 64 keys of both rows.
  static_assert(kCoreWaves == 8 && G == 2, "DMA job split assumes 8 waves and 2 rows");
  // Each source walks forward by one stage per call: K rows by kKT * kD
  // elements, V^T rows by kKT keys, the bias by 4 key blocks (kKT * 16).
  const bf16* kv_src[2];
  int kv_step[2];
  unsigned kv_lds[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int job = w + 8 * u, r = job >> 3, kind = (job >> 2) & 1, quarter = job & 3;
    if (kind == 0) {
      const int key = 16 * quarter + (l >> 2), c = (l & 3) ^ ((key >> 2) & 3);
      kv_src[u] = kb[r] + key * kD + 8 * c;
      kv_step[u] = kKT * kD;
    } else {
      const int d = 8 * quarter + (l >> 3), c = (l & 7) ^ ((d >> 1) & 7);
      kv_src[u] = vb[r] + (int64_t)d * np + 8 * c;
      kv_step[u] = kKT;
    }
    kv_lds[u] = (kind == 0 ? kOffK : kOffV) + r * kTileBytes + 1024 * quarter;
  }
  const bf16* tb_src = L.tb + tb_offset(np, h, q0, 0) + 8 * l;  // + 256 per 16-key block
  const int i_mb = min(i0 + (l >> 4), n - 1);
  const float* mb_src = L.mb + (int64_t)i_mb * np + 4 * lq;
  auto dma_stage = [&](int buf, int stage_k0) {
    const unsigned base = lds0 + buf * kStageBytes;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      lds_dma16(kv_src[u], __builtin_amdgcn_readfirstlane(base + kv_lds[u]));
      kv_src[u] += kv_step[u];
    }
#pragma unroll
    for (int hb = 0; hb < 2; ++hb)
      lds_dma16(tb_src + 16 * 32 * hb,
                __builtin_amdgcn_readfirstlane(base + kOffBias + w * kBiasWaveBytes + 1024 * hb));
    tb_src += 16 * kKT;
    if ((MASKED || (KEYMASK && stage_k0 >= mask_k0)) && w == 0 && l < 32)
      lds_dma16(mb_src, __builtin_amdgcn_readfirstlane(base + kOffMb));
    mb_src += kKT;
  };

  // O^T tiles (d 0..15, 16..31) and the row sum l, which an MFMA with an
  // all-ones A operand accumulates from the same bf16 P that multiplies V.
  f32x4 o[G][2], ls[G];
  // m: the max offset subtracted from this lane's scores.  Unmasked rows
  // start the QK^T MFMA from C = -m (mneg), so the subtraction is free.
  float m[G];
  f32x4 mneg[G];
#pragma unroll
  for (int r = 0; r < G; ++r) {
    o[r][0] = o[r][1] = ls[r] = f32x4{0.f, 0.f, 0.f, 0.f};
    m[r] = MASKED ? -INFINITY : 0.f;
    mneg[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // ident: A operand with A[key][kk] = (kk == key) for kk < 16, so that one
  // MFMA with the bias tile as B adds bias^T to S^T.
  bf16x8 ones, ident = {};
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (bf16)1.f;
  if (g == (lq >> 3)) ident[lq & 7] = (bf16)1.f;

  // Per-lane LDS read offsets (bytes) inside a stage buffer.
  const int k_rd = kOffK + (4 * lq + (g ^ ((lq >> 2) & 3))) * 16;  // + 1024 j (16 keys) + r tile
  const int b_rd = kOffBias + w * kBiasWaveBytes + 16 * (l & 31);   // + 512 j

  dma_stage(0, 0);
  wait_vm0();
  __syncthreads();
  for (int k0 = 0; k0 < nk; k0 += kKT) {
    const int cur = (k0 / kKT) & 1;
    const bool more = k0 + kKT < nk;
    if (more) dma_stage(cur ^ 1, k0 + kKT);
    const char* sb = lds + cur * kStageBytes;
    // S^T for all rows first, so the scheduler can overlap one row's MFMAs
    // with another row's max / exp work inside one basic block.
    f32x4 s[G][4];
    float mt[G];
    // Triangle-bias B tile j: lanes of groups 0 and 1 hold keys 16j + 8g .. +7
    // of their query; groups 2 and 3 read the same bytes, which ident
    // multiplies by zero (the bias is finite).
    if constexpr (SPEC) {
      const bool mstage = KEYMASK && k0 >= mask_k0;  // wave-uniform
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x4 bc = mfma16(ident, *(const bf16x8*)(sb + b_rd + 512 * j), mneg[0]);
#pragma unroll
        for (int r = 0; r < G; ++r) {
          f32x4 c = bc;
          if (mstage) c += *(const f32x4*)(sb + kOffMb + r * kKT * 4 + (16 * j + 4 * g) * 4);
          s[r][j] = mfma16(*(const bf16x8*)(sb + k_rd + r * kTileBytes + 1024 * j), qf[r], c);
        }
      }
    }
#pragma unroll
    for (int r = 0; r < G; ++r) {
      if constexpr (!SPEC) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 c = MASKED ? *(const f32x4*)(sb + kOffMb + r * kKT * 4 + (16 * j + 4 * g) * 4) : mneg[r];
          s[r][j] = mfma16(*(const bf16x8*)(sb + k_rd + r * kTileBytes + 1024 * j), qf[r], c);
          s[r][j] = mfma16(ident, *(const bf16x8*)(sb + b_rd + 512 * j), s[r][j]);
        }
      }
      // This lane's max over its 16 keys (a v_max3 tree: 5 + 2 + 1); the max
      // over all keys of a query (4 lanes) is only needed when some lane
      // crosses the lazy threshold.  Speculative passes need it only once.
      if (!SPEC || k0 == 0) {
        const f32x4* sr = s[r];
        const float a0 = max3f(sr[0][0], sr[0][1], sr[0][2]), a1 = max3f(sr[0][3], sr[1][0], sr[1][1]);
        const float a2 = max3f(sr[1][2], sr[1][3], sr[2][0]), a3 = max3f(sr[2][1], sr[2][2], sr[2][3]);
        const float a4 = max3f(sr[3][0], sr[3][1], sr[3][2]);
        mt[r] = fmaxf(max3f(a0, a1, a2), max3f(a3, a4, sr[3][3]));
      }
    }
    bool grow = false;
#pragma unroll
    for (int r = 0; r < G; ++r) grow |= SPEC ? false : MASKED ? mt[r] > m[r] + kLazy : mt[r] > kLazy;
    auto query_max = [](float v) {
      v = fmaxf(v, __shfl_xor(v, 16, kWave));
      return fmaxf(v, __shfl_xor(v, 32, kWave));
    };
    if ((!MASKED && k0 == 0) || __any(grow)) {  // wave-uniform; rare after the first stages
      float mall = mt[0];
#pragma unroll
      for (int r = 1; r < G; ++r) mall = fmaxf(mall, mt[r]);
      const float qshared = SPEC ? query_max(mall) : 0.f;
#pragma unroll
      for (int r = 0; r < G; ++r) {
        const float qmax = SPEC ? qshared : query_max(mt[r]);
        float mn;
        if (MASKED)
          mn = fmaxf(m[r], qmax);
        else  // first stage: start from the tile max; later: raise the offset by the excess
          mn = k0 == 0 ? qmax : m[r] + fmaxf(qmax, 0.f);
        const float delta = m[r] - mn;
        if (MASKED || k0 != 0) {
          const float alpha = __builtin_amdgcn_exp2f(delta);
          o[r][0] = o[r][0] * alpha;
          o[r][1] = o[r][1] * alpha;
          ls[r] = ls[r] * alpha;
        }
        m[r] = mn;
        if (!MASKED) {
          mneg[r] = f32x4{-mn, -mn, -mn, -mn};
#pragma unroll
          for (int j = 0; j < 4; ++j) s[r][j] = s[r][j] + delta;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < G; ++r) {
      if (MASKED) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s[r][j] = s[r][j] - m[r];
      }
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        // P^T operand for keys 32st..32st+31: element e <-> key 32st + 16(e/4) + 4g + e%4
        bf16x8 pf;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pf[e] = (bf16)__builtin_amdgcn_exp2f(s[r][2 * st][e]);
          pf[4 + e] = (bf16)__builtin_amdgcn_exp2f(s[r][2 * st + 1][e]);
        }
        ls[r] = mfma16(ones, pf, ls[r]);
#pragma unroll
        for (int mt2 = 0; mt2 < 2; ++mt2) {
          // V^T rows d = 16 mt2 + l%16 hold the same key order (stored permuted)
          const int d = 16 * mt2 + lq, c = 4 * st + g;
          const bf16x8 vf =
              *(const bf16x8*)(sb + kOffV + r * kTileBytes + (8 * d + (c ^ ((d >> 1) & 7))) * 16);
          o[r][mt2] = mfma16(vf, pf, o[r][mt2]);
        }
      }
    }
    wait_vm0();  // this wave's DMAs of the next stage
    __syncthreads();
  }
  if (SPEC) {
    // Exponent-field tests (this file builds with -fno-honor-nans, so no
    // floating-point NaN compares): every row sum in [2^-60, 2^101), every output finite.
    bool ok = true;
#pragma unroll
    for (int r = 0; r < G; ++r) {
      const unsigned ex = (__float_as_uint(ls[r][0]) >> 23) & 0xFF;
      ok &= ex <= 127 + 100 && ex >= 127 - 60;
#pragma unroll
      for (int mt2 = 0; mt2 < 2; ++mt2)
#pragma unroll
        for (int e = 0; e < 4; ++e) ok &= (__float_as_uint(o[r][mt2][e]) & 0x7F800000u) != 0x7F800000u;
    }
    if (__syncthreads_or(!ok)) return false;
  }
  const int q = q0 + lq;
#pragma unroll
  for (int r = 0; r < G; ++r) {
    if (i0 + r < n && q < n) {
      const float inv = __builtin_amdgcn_rcpf(ls[r][0]);
      bf16* dst = L.o + ((int64_t)(i0 + r) * n + q) * kC + h * kD + 4 * g;
#pragma unroll
      for (int mt2 = 0; mt2 < 2; ++mt2) {
        const bf16x4 pk = {(bf16)(o[r][mt2][0] * inv), (bf16)(o[r][mt2][1] * inv), (bf16)(o[r][mt2][2] * inv),
                           (bf16)(o[r][mt2][3] * inv)};
        *(bf16x4*)(dst + 16 * mt2) = pk;
      }
    }
  }
  return true;
}

// Rows with every key masked: the mask bias (-1e9 log2 e) swamps every
// score, so upstream's softmax is uniform over the n keys and each query's
// output is the mean of v over them (the masked path gives the same: every
// score rounds to the mask bias, p = 1).  Keys past n hold v = 0.  Each wave
// writes its 16 queries; lane (d = l % 32, half = l / 32) sums dim d over
// half of the keys.
__device__ __forceinline__ void uniform_rows(const Layout& L, int i0, int h, int q0) {
  const int n = L.n, np = L.np, l = lane_id(), d = l & 31, half = l >> 5;
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    const int i = i0 + r;
    if (i >= n) break;
    const bf16* vrow = L.vt + (((int64_t)i * kH + h) * kD + d) * np;
    float acc = 0.f;
    for (int k = 8 * half; k < np; k += 16) {
      const bf16x8 v = gload8(vrow + k);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc += (float)v[e];
    }
    acc += __shfl_xor(acc, 32, kWave);
    const bf16 mean = (bf16)(acc * (1.f / n));
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int q = q0 + 8 * half + u;
      if (q < n) L.o[((int64_t)i * n + q) * kC + h * kD + d] = mean;
    }
  }
}

// Two 8-wave blocks per CU need <= 128 VGPRs; one register more would leave a
// single block per CU, which measured 1.5-2.3x slower, so the budget is pinned.
__global__ __launch_bounds__(kCoreThreads) __attribute__((amdgpu_waves_per_eu(4))) void triattn_core_kernel(Layout L) {
  __shared__ __attribute__((aligned(16))) char stage_lds[2 * kStageBytes];
  const int n = L.n, np = L.np;
  const int qtiles = core_qtiles(n);
  const int cpx = core_cols_per_xcd(n);
  const int bid = blockIdx.x;
  const int idx = bid >> 3;
  const int col = (bid & 7) * cpx + idx % cpx, ig = idx / cpx;
  if (col >= kH * qtiles) return;  // uniform over the block
  const int h = col / qtiles, qt = col % qtiles;
  const int t = threadIdx.x, w = t >> 6;
  const int i0 = ig * kRows;
  const int q0 = qt * kCoreQ + 16 * w;  // this wave's 16 queries (< np: np is a multiple of kCoreQ)

  // Row classes from the projection's per-tile key spans: per row, the first
  // masked key and the last open one.  Every wave reduces the same entries
  // (shuffles, no barrier).
  bool any_mask = false, suffix = true, all_closed = true;
  int kend = 0, mask_from = n;
  {
    const int l = t & (kWave - 1), tiles = np / kP1;
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int2* span = L.keyspan + (int64_t)min(i0 + r, n - 1) * tiles;  // rows past n repeat row n-1
      int fm = n, lo = -1;
      for (int e = l; e < tiles; e += kWave) {
        const int2 v = span[e];
        fm = min(fm, v.x);
        lo = max(lo, v.y);
      }
#pragma unroll
      for (int d = 32; d >= 1; d >>= 1) {
        fm = min(fm, __shfl_xor(fm, d, kWave));
        lo = max(lo, __shfl_xor(lo, d, kWave));
      }
      any_mask |= fm < n;
      all_closed &= lo < 0 && fm >= 0;  // no open key, and every key closed by a 0 mask (no fractional one)
      suffix &= lo >= 0 && lo < fm;  // some open key, and every open key before every masked one
      kend = max(kend, fm);          // keys from here on are masked in every row (or past n)
      mask_from = min(mask_from, fm);
    }
  }
  const int nk = (n + kKT - 1) / kKT * kKT;
  if (all_closed) {
    uniform_rows(L, i0, h, q0);
  } else if (!any_mask) {
    if (!core_rows<false, true>(L, i0, h, q0, stage_lds, nk, nk))
      // a score rose far above the first stage's max: redo the block with the tracked max
      core_rows<false, false>(L, i0, h, q0, stage_lds, nk, nk);
  } else if (!suffix || !core_rows<false, true, true>(L, i0, h, q0, stage_lds, (kend + kKT - 1) / kKT * kKT,
                                                      mask_from / kKT * kKT)) {
    core_rows<true, false>(L, i0, h, q0, stage_lds, nk, nk);
  }
}

// ------------------------------------------------------------------ K3
// Persistent and weight-stationary; a tile is 64 positions (i, j0..j0+63) of
// the row frame.  Input rows stay in registers from the prefetch to the
// residual add, so x is read once; results are re-laid out through LDS
// (ybuf), where the residual is added.  Tile k's rows are stored from ybuf in
// iteration k+1, before the next prefetch: vmcnt counts stores in issue
// order, so the wait for that prefetch does not wait for fresh stores.
// kScaled: the module output of frame row i is multiplied by row_scale[i]
// before it is written or added (PairformerLayer's row / column dropout mask:
// frame row i is z's row i for the starting node and z's column i for the
// ending node).
constexpr int kP3 = 64;

template <typename TIn, bool kScaled, bool starting>
__global__ __launch_bounds__(256, 2) void triattn_out_kernel(const TIn* x, const float* __restrict__ ln_w,
                                                             const float* __restrict__ ln_b, float eps,
                                                             const bf16* __restrict__ w_g,
                                                             const float* __restrict__ b_g,
                                                             const bf16* __restrict__ w_o,
                                                             const float* __restrict__ b_o, void* out,
                                                             int out_mode, const float* __restrict__ row_scale,
                                                             Layout L) {
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kP3 * kLdsRow];
  __shared__ __attribute__((aligned(16))) float ybuf[kP3 * kYRow];  // fp32 result rows
  bf16* xg = smem;                   // LN(x'), pairs x channels
  bf16* xo = smem + kP3 * kLdsRow;   // attention output, then o * gate
  const int n = L.n;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6, c0 = 32 * w, ch = c0 + (l & 31);
  const int hw = t >> 5, hl = t & 31;
  const LnAffine aff = ln_affine(ln_w, ln_b, hl);
  const int tiles_x = (n + kP3 - 1) / kP3, total = n * tiles_x;
  const bool x_in_regs = out_mode == kOutResidual || (const void*)x == out;

  bf16x8 wg[8], wo[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    wg[ks] = frag(w_g, kC, c0, ks);
    wo[ks] = frag(w_o, kC, c0, ks);
  }
  const float bg = b_g[ch], bo = b_o[ch];

  // Rows past n re-read row n-1 (unconditional loads) and are not stored.
  constexpr int kRowsPer = kP3 / 8;
  f32x4 px[kRowsPer];
  bf16x4 po[kRowsPer];
  float prs = 1.f;
  auto fetch = [&](int tile) {
    const int i = tile / tiles_x, j0 = (tile % tiles_x) * kP3;
    if constexpr (kScaled) prs = row_scale[i];
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      const int j = min(j0 + hw + 8 * u, n - 1);
      px[u] = load4(xrow(x, n, starting, i, j) + 4 * hl);
      po[u] = *(const bf16x4*)(L.o + ((int64_t)i * n + j) * kC + 4 * hl);
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
        const int64_t off = (starting ? (int64_t)i * n + j : (int64_t)j * n + i) * kC + 4 * hl;
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
    for (int u = 0; u < kRowsPer; ++u) xc[u] = px[u];
    ln128_half_rows(px, aff, eps);  // px is fetched again after the barrier
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      bf16x4 o = {(bf16)px[u][0], (bf16)px[u][1], (bf16)px[u][2], (bf16)px[u][3]};
      *(bf16x4*)(xg + (hw + 8 * u) * kLdsRow + 4 * hl) = o;
      *(bf16x4*)(xo + (hw + 8 * u) * kLdsRow + 4 * hl) = po[u];
    }
    if (prev >= 0) store_rows(prev);
    __syncthreads();
    if (tile + (int)gridDim.x < total) fetch(tile + gridDim.x);

    // Gate: D[pair][ch], lane = channel.  Each (pair, channel) of xo is owned
    // by exactly one lane, so the in-place multiply needs no barrier.
#pragma unroll
    for (int nt = 0; nt < kP3 / 32; ++nt) {
      f32x16 acc = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) acc = mfma32(frag(xg, kLdsRow, nt * 32, ks), wg[ks], acc);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        bf16* e = xo + (nt * 32 + drow(r, l)) * kLdsRow + ch;
        *e = (bf16)((float)*e * sigmoid_f(acc[r] + bg));
      }
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < kP3 / 32; ++nt) {
      f32x16 acc = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) acc = mfma32(frag(xo, kLdsRow, nt * 32, ks), wo[ks], acc);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float y = rbf(acc[r] + bo);
        if constexpr (kScaled) y *= rs;
        ybuf[(nt * 32 + drow(r, l)) * kYRow + ch] = y;
      }
    }
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

Layout make_layout(void* ws, int n) {
  Layout L;
  L.n = n;
  L.np = (int)round_up(n, kPad);
  const int64_t e = qkv_elems(L.np);
  char* p = (char*)ws;
  L.q = (bf16*)p;
  p += e * sizeof(bf16);
  L.k = (bf16*)p;
  p += e * sizeof(bf16);
  L.vt = (bf16*)p;
  p += e * sizeof(bf16);
  L.o = (bf16*)p;
  p += round_up((int64_t)n * n * kC * sizeof(bf16), 256);
  L.tb = (tb_t*)p;
  p += (int64_t)kH * L.np * L.np * sizeof(tb_t);
  L.mb = (float*)p;
  p += (int64_t)L.np * L.np * 4;
  L.keyspan = (int2*)p;
  return L;
}

template <typename TIn>
int run(const TIn* x, const float* mask, int n, int starting, float inf, const float* ln_w, const float* ln_b,
        float eps, const bf16* w_proj, const bf16* w_g, const float* b_g, const bf16* w_o, const float* b_o,
        void* out, int out_mode, const float* row_scale, void* ws, int stages, hipStream_t st) {
  Layout L = make_layout(ws, n);
  if (stages & 1) {
    const int total = L.np * (L.np / kP1);
    const int grid = total < 2 * device_cu_count() ? total : 2 * device_cu_count();
    if (starting)
      triattn_proj_kernel<TIn, true><<<dim3(grid), 256, 0, st>>>(x, mask, ln_w, ln_b, eps, w_proj, inf, L);
    else
      triattn_proj_kernel<TIn, false><<<dim3(grid), 256, 0, st>>>(x, mask, ln_w, ln_b, eps, w_proj, inf, L);
    if (int rc = check_launch("triattn_proj")) return rc;
  }
  if (stages & 2) {
    triattn_core_kernel<<<dim3((unsigned)(8ll * core_cols_per_xcd(n) * core_row_groups(n))), kCoreThreads, 0, st>>>(L);
    if (int rc = check_launch("triattn_core")) return rc;
  }
  if (stages & 4) {
    const int total = n * ((n + kP3 - 1) / kP3);
    const int grid = total < 2 * device_cu_count() ? total : 2 * device_cu_count();
    auto launch_out = [&](auto scaled, auto start) {
      triattn_out_kernel<TIn, decltype(scaled)::value, decltype(start)::value>
          <<<dim3(grid), 256, 0, st>>>(x, ln_w, ln_b, eps, w_g, b_g, w_o, b_o, out, out_mode, row_scale, L);
    };
    using T = std::true_type;
    using F = std::false_type;
    if (row_scale)
      starting ? launch_out(T{}, T{}) : launch_out(T{}, F{});
    else
      starting ? launch_out(F{}, T{}) : launch_out(F{}, F{});
    if (int rc = check_launch("triattn_out")) return rc;
  }
  return BMX_OK;
}

}  // namespace

extern "C" {

size_t bmx_triattn_workspace_bytes(int64_t n) {
  if (n <= 0) return 0;
  int64_t np = round_up(n, kPad);
  return (size_t)(3 * qkv_elems((int)np) * 2 + round_up(n * n * kC * 2, 256) + (int64_t)kH * np * np * (int64_t)sizeof(tb_t) +
                  np * np * 4 + np * (np / kP1) * (int64_t)sizeof(int2));
}

int bmx_triattn_fwd(const void* x, int x_dtype, const float* mask, int64_t n, int starting, float inf,
                    const float* ln_w, const float* ln_b, float eps, const void* w_proj, const void* w_g,
                    const float* b_g, const void* w_o, const float* b_o, void* out, int out_mode,
                    const float* row_scale, void* workspace, size_t workspace_bytes, int stages, hipStream_t stream) {
  BMX_REQUIRE(n >= 0 && n <= 8192, "bmx_triattn_fwd: n must be in [0, 8192] (got %lld)", (long long)n);
  BMX_REQUIRE(x_dtype == kF32 || x_dtype == kBF16, "bmx_triattn_fwd: x dtype must be fp32 or bf16");
  BMX_REQUIRE(out_mode >= 0 && out_mode <= 3,
              "bmx_triattn_fwd: out_mode must be 0 (bf16), 1 (fp32), 2 (fp32 +=) or 3 (fp32 x + y)");
  BMX_REQUIRE(out_mode != 2 || x_dtype == kF32, "bmx_triattn_fwd: residual mode needs fp32 x");
  BMX_REQUIRE(stages >= 1 && stages <= 7, "bmx_triattn_fwd: stages must be a non-empty subset of 1|2|4");
  BMX_REQUIRE(eps > 0.f && inf > 0.f, "bmx_triattn_fwd: eps and inf must be positive");
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(x && ln_w && ln_b && w_proj && w_g && b_g && w_o && b_o && out, "bmx_triattn_fwd: null pointer");
  BMX_REQUIRE(workspace && workspace_bytes >= bmx_triattn_workspace_bytes(n),
              "bmx_triattn_fwd: workspace too small (%zu < %zu bytes)", workspace_bytes,
              bmx_triattn_workspace_bytes(n));
  BMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)workspace % 256 == 0 && (uintptr_t)w_proj % 16 == 0 &&
                  (uintptr_t)w_g % 16 == 0 && (uintptr_t)w_o % 16 == 0,
              "bmx_triattn_fwd: x and weights must be 16-byte aligned, workspace 256-byte aligned");
  if (x_dtype == kF32)
    return run<float>((const float*)x, mask, (int)n, starting, inf, ln_w, ln_b, eps, (const bf16*)w_proj,
                      (const bf16*)w_g, b_g, (const bf16*)w_o, b_o, out, out_mode, row_scale, workspace, stages,
                      stream);
  return run<bf16>((const bf16*)x, mask, (int)n, starting, inf, ln_w, ln_b, eps, (const bf16*)w_proj,
                   (const bf16*)w_g, b_g, (const bf16*)w_o, b_o, out, out_mode, row_scale, workspace, stages, stream);
}

int bmx_triattn_proj_rows(void) { return kProjRows; }

}  // extern "C"
