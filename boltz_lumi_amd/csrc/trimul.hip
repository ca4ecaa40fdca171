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
#include "bmx_common.h"

using namespace bmx;

namespace {

constexpr int kTP = 128;               // pairs per K1 / K3 block
constexpr int kStageRow = kTP + 8;     // staged plane rows (bf16)
constexpr int kPlaneTile = 128;        // plane padding granularity

// ------------------------------------------------------------------ K1
__global__ __launch_bounds__(256) void trimul_proj_kernel(const float* __restrict__ x, const float* __restrict__ mask,
                                                          const float* __restrict__ ln_w,
                                                          const float* __restrict__ ln_b, float eps,
                                                          const bf16* __restrict__ w_in, bf16* __restrict__ a_pl,
                                                          bf16* __restrict__ b_pl, int n, int np, int outgoing) {
  // X tile [kTP][kLdsRow] aliases the front of the output staging area
  // stage[2][kC][kStageRow].
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kC * kStageRow];
  bf16* xt = smem;
  const int rp = blockIdx.y;
  const int t0 = blockIdx.x * kTP;
  const int l = lane_id(), w = threadIdx.x >> 6;

  auto row_ptr = [&](int p) -> const float* {
    int t = t0 + p;
    if (rp >= n || t >= n) return nullptr;
    int64_t pair = outgoing ? (int64_t)rp * n + t : (int64_t)t * n + rp;
    return x + pair * kC;
  };
  ln_rows_to_lds<kTP, float>(row_ptr, ln_w, ln_b, eps, xt);
  __syncthreads();

  // Wave w owns channels [32w, 32w+32) of a and of b.  Orientation: D[ch][pair]
  // (A = weight rows, B = normalised pairs), so lane l holds pair l%32.
  const int c0 = 32 * w;
  uint32_t res[2][4][8];  // [a|b][pair tile][packed bf16 pairs of registers]
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    bf16x8 wp[8], wg[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      wp[ks] = frag(w_in, kC, half * kC + c0, ks);
      wg[ks] = frag(w_in, kC, 2 * kC + half * kC + c0, ks);
    }
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      f32x16 ap = zero16(), ag = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        bf16x8 xf = frag(xt, kLdsRow, nt * 32, ks);
        ap = mfma32(wp[ks], xf, ap);
        ag = mfma32(wg[ks], xf, ag);
      }
      const int t = t0 + nt * 32 + (l & 31);
      float m = 0.f;
      if (rp < n && t < n) m = mask[outgoing ? (int64_t)rp * n + t : (int64_t)t * n + rp];
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float v0 = rbf(rbf(rbf(ap[r]) * rbf(sigmoid_f(rbf(ag[r])))) * m);
        float v1 = rbf(rbf(rbf(ap[r + 1]) * rbf(sigmoid_f(rbf(ag[r + 1])))) * m);
        bf16x2 pk = {(bf16)v0, (bf16)v1};
        res[half][nt][r >> 1] = __builtin_bit_cast(uint32_t, pk);
      }
    }
  }
  __syncthreads();  // X tile is dead; reuse LDS as the staging area
#pragma unroll
  for (int half = 0; half < 2; ++half)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        bf16x2 pk = __builtin_bit_cast(bf16x2, res[half][nt][r >> 1]);
        int ch = c0 + drow(r, l);
        smem[(half * kC + ch) * kStageRow + nt * 32 + (l & 31)] = pk[r & 1];
      }
  __syncthreads();
  const int64_t plane = (int64_t)np * np;
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    int idx = threadIdx.x + 256 * u;
    int half = idx >> 11, ch = (idx >> 4) & 127, chunk = idx & 15;
    bf16x8 v = *(const bf16x8*)(smem + (half * kC + ch) * kStageRow + chunk * 8);
    bf16* dst = (half ? b_pl : a_pl) + ch * plane + (int64_t)rp * np + t0 + chunk * 8;
    *(bf16x8*)dst = v;
  }
}

// ------------------------------------------------------------------ K2
// Batched NT GEMM over channels: O_c[m][n] = sum_k A_c[m][k] * B_c[n][k].
template <int BM, int BN, int BK, int WM, int WN>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void trimul_contract_kernel(
    const bf16* __restrict__ A, const bf16* __restrict__ B, bf16* __restrict__ O, int np, int tiles_n,
    int tiles_per_ch) {
  constexpr int kWavesN = BN / WN;
  constexpr int kThreads = (BM / WM) * kWavesN * 64;
  constexpr int kLd = BK + 8;
  constexpr int kMi = WM / 32, kNi = WN / 32;
  constexpr int kChunksA = BM * BK / 8 / kThreads;
  constexpr int kChunksB = BN * BK / 8 / kThreads;
  static_assert(kChunksA * kThreads * 8 == BM * BK && kChunksB * kThreads * 8 == BN * BK, "tile/thread mismatch");
  __shared__ __attribute__((aligned(16))) bf16 As[2][BM * kLd];
  __shared__ __attribute__((aligned(16))) bf16 Bs[2][BN * kLd];

  // Blocks are dispatched round-robin over the 8 XCDs; give every XCD whole
  // channels so the channel's operand planes stay in that XCD's L2.
  const int b = blockIdx.x;
  const int xcd = b & 7, idx = b >> 3;
  const int c = xcd + 8 * (idx / tiles_per_ch);
  const int tile = idx % tiles_per_ch;
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int64_t plane = (int64_t)np * np;
  const bf16* Ac = A + c * plane + (int64_t)tm * BM * np;
  const bf16* Bc = B + c * plane + (int64_t)tn * BN * np;

  const int t = threadIdx.x, l = lane_id(), wv = t >> 6;
  const int wm0 = (wv / kWavesN) * WM, wn0 = (wv % kWavesN) * WN;

  bf16x8 ra[kChunksA], rb[kChunksB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int u = 0; u < kChunksA; ++u) {
      int i = t + kThreads * u, row = i / (BK / 8), col = (i % (BK / 8)) * 8;
      ra[u] = *(const bf16x8*)(Ac + (int64_t)row * np + k0 + col);
    }
#pragma unroll
    for (int u = 0; u < kChunksB; ++u) {
      int i = t + kThreads * u, row = i / (BK / 8), col = (i % (BK / 8)) * 8;
      rb[u] = *(const bf16x8*)(Bc + (int64_t)row * np + k0 + col);
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kChunksA; ++u) {
      int i = t + kThreads * u, row = i / (BK / 8), col = (i % (BK / 8)) * 8;
      *(bf16x8*)(&As[buf][row * kLd + col]) = ra[u];
    }
#pragma unroll
    for (int u = 0; u < kChunksB; ++u) {
      int i = t + kThreads * u, row = i / (BK / 8), col = (i % (BK / 8)) * 8;
      *(bf16x8*)(&Bs[buf][row * kLd + col]) = rb[u];
    }
  };

  f32x16 acc[kMi][kNi];
#pragma unroll
  for (int i = 0; i < kMi; ++i)
#pragma unroll
    for (int j = 0; j < kNi; ++j) acc[i][j] = zero16();

  const int kt_count = np / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < kt_count; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < kt_count) gload((kt + 1) * BK);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8 af[kMi], bfr[kNi];
#pragma unroll
      for (int i = 0; i < kMi; ++i) af[i] = frag(As[cur], kLd, wm0 + 32 * i, ks);
#pragma unroll
      for (int j = 0; j < kNi; ++j) bfr[j] = frag(Bs[cur], kLd, wn0 + 32 * j, ks);
#pragma unroll
      for (int i = 0; i < kMi; ++i)
#pragma unroll
        for (int j = 0; j < kNi; ++j) acc[i][j] = mfma32(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < kt_count) sstore(cur ^ 1);
    __syncthreads();
  }

  bf16* Oc = O + c * plane + (int64_t)(tm * BM) * np + tn * BN;
#pragma unroll
  for (int i = 0; i < kMi; ++i)
#pragma unroll
    for (int j = 0; j < kNi; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        int m = wm0 + 32 * i + drow(r, l);
        int nn = wn0 + 32 * j + (l & 31);
        Oc[(int64_t)m * np + nn] = (bf16)acc[i][j][r];
      }
}

// ------------------------------------------------------------------ K3
__global__ __launch_bounds__(256) void trimul_out_kernel(const float* x, const bf16* __restrict__ o_pl,
                                                         const float* __restrict__ in_w, const float* __restrict__ in_b,
                                                         float eps_in, const float* __restrict__ out_w,
                                                         const float* __restrict__ out_b, float eps_out,
                                                         const bf16* __restrict__ w_pout,
                                                         const bf16* __restrict__ w_gout, void* out,
                                                         int out_mode, int n, int np) {
  __shared__ __attribute__((aligned(16))) bf16 xo[kTP * kLdsRow];  // LN_out(O), pairs x channels
  __shared__ __attribute__((aligned(16))) bf16 xg[kTP * kLdsRow];  // LN_in(x), pairs x channels
  const int i = blockIdx.y, j0 = blockIdx.x * kTP;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6;
  const int64_t plane = (int64_t)np * np;

  // Product tile O[c][i][j0..j0+127] -> xo[p][c] (transposed through LDS).
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    int idx = t + 256 * u, c = idx >> 4, chunk = idx & 15;
    bf16x8 v = *(const bf16x8*)(o_pl + c * plane + (int64_t)i * np + j0 + chunk * 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) xo[(chunk * 8 + e) * kLdsRow + c] = v[e];
  }
  auto row_ptr = [&](int p) -> const float* {
    return (j0 + p < n) ? x + ((int64_t)i * n + j0 + p) * kC : nullptr;
  };
  ln_rows_to_lds<kTP, float>(row_ptr, in_w, in_b, eps_in, xg);
  __syncthreads();
  {
    const int hw = t >> 5, hl = t & 31;
#pragma unroll 4
    for (int u = 0; u < kTP / 8; ++u) {
      bf16* row = xo + (hw + 8 * u) * kLdsRow + 4 * hl;
      f32x4 v = {(float)row[0], (float)row[1], (float)row[2], (float)row[3]};
      f32x4 y = ln128_half(v, out_w, out_b, hl, eps_out);
      bf16x4 o = {(bf16)y[0], (bf16)y[1], (bf16)y[2], (bf16)y[3]};
      *(bf16x4*)row = o;
    }
  }
  __syncthreads();

  // D[pair][ch]: A = normalised pairs, B = weight rows; lane l holds channel c0 + l%32.
  const int c0 = 32 * w;
  bf16x8 wp[8], wg[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    wp[ks] = frag(w_pout, kC, c0, ks);
    wg[ks] = frag(w_gout, kC, c0, ks);
  }
  const int ch = c0 + (l & 31);
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    f32x16 ay = zero16(), ag = zero16();
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      ay = mfma32(frag(xo, kLdsRow, nt * 32, ks), wp[ks], ay);
      ag = mfma32(frag(xg, kLdsRow, nt * 32, ks), wg[ks], ag);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      int j = j0 + nt * 32 + drow(r, l);
      if (j >= n) continue;
      float y = rbf(rbf(ay[r]) * rbf(sigmoid_f(rbf(ag[r]))));
      int64_t o = ((int64_t)i * n + j) * kC + ch;
      if (out_mode == 0)
        ((bf16*)out)[o] = (bf16)y;
      else if (out_mode == 1)
        ((float*)out)[o] = y;
      else if (out_mode == 2)
        ((float*)out)[o] += y;
      else
        ((float*)out)[o] = x[o] + y;
    }
  }
}

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

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
                   int out_mode, void* workspace, size_t workspace_bytes, int stages, hipStream_t stream) {
  BMX_REQUIRE(n >= 0 && n <= 16384, "bmx_trimul_fwd: n must be in [0, 16384] (got %lld)", (long long)n);
  BMX_REQUIRE(out_mode >= 0 && out_mode <= 3,
              "bmx_trimul_fwd: out_mode must be 0 (bf16), 1 (fp32), 2 (fp32 +=) or 3 (fp32 x + y)");
  BMX_REQUIRE(stages >= 1 && stages <= 7, "bmx_trimul_fwd: stages must be a non-empty subset of 1|2|4");
  BMX_REQUIRE(eps_in > 0.f && eps_out > 0.f, "bmx_trimul_fwd: eps must be positive");
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(x && mask && norm_in_w && norm_in_b && w_in && norm_out_w && norm_out_b && w_pout && w_gout && out,
              "bmx_trimul_fwd: null pointer");
  BMX_REQUIRE(workspace && workspace_bytes >= bmx_trimul_workspace_bytes(n),
              "bmx_trimul_fwd: workspace too small (%zu < %zu bytes)", workspace_bytes,
              bmx_trimul_workspace_bytes(n));
  BMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)workspace % 16 == 0 && (uintptr_t)w_in % 16 == 0 &&
                  (uintptr_t)w_pout % 16 == 0 && (uintptr_t)w_gout % 16 == 0,
              "bmx_trimul_fwd: x, weights and workspace must be 16-byte aligned");
  const int ni = (int)n;
  const int np = (int)round_up(n, kPlaneTile);
  const int64_t plane = (int64_t)np * np * kC;
  bf16* a_pl = (bf16*)workspace;
  bf16* b_pl = a_pl + plane;
  bf16* o_pl = b_pl + plane;

  if (stages & 1) {
    trimul_proj_kernel<<<dim3(np / kTP, np), 256, 0, stream>>>(x, mask, norm_in_w, norm_in_b, eps_in,
                                                                (const bf16*)w_in, a_pl, b_pl, ni, np, outgoing);
    if (int rc = check_launch("trimul_proj")) return rc;
  }
  if (stages & 2) {
    constexpr int BM = 128, BN = 128, BK = 64;
    const int tiles_n = np / BN, tiles_per_ch = (np / BM) * tiles_n;
    trimul_contract_kernel<BM, BN, BK, 64, 64><<<dim3(kC * tiles_per_ch), 256, 0, stream>>>(
        a_pl, b_pl, o_pl, np, tiles_n, tiles_per_ch);
    if (int rc = check_launch("trimul_contract")) return rc;
  }
  if (stages & 4) {
    trimul_out_kernel<<<dim3((ni + kTP - 1) / kTP, ni), 256, 0, stream>>>(
        x, o_pl, norm_in_w, norm_in_b, eps_in, norm_out_w, norm_out_b, eps_out, (const bf16*)w_pout,
        (const bf16*)w_gout, out, out_mode, ni, np);
    if (int rc = check_launch("trimul_out")) return rc;
  }
  return BMX_OK;
}

}  // extern "C"
