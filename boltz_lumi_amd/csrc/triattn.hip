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
//  K2 triattn_core   one block per (row i, head h, 128 queries); per 32-key
//                    tile S^T = K Q^T + (tb + mb)^T with the bias as the MFMA C
//                    operand, online softmax in base 2 (fp32), O^T += V^T P^T
//                    with P kept in registers (bf16).
//  K3 triattn_out    o * sigmoid(linear_g(LN(x')) + b_g) -> linear_o + b_o, then
//                    write or add into the fp32 residual in place.
//
// Workspace (np = round_up(n, 128)):
//   q[i][h][j][d], k[i][h][j][d], vt[i][h][d][j]  bf16, i < np, j < np
//   tb[h][q][k] fp32 (k >= n is -inf), mb[i][k] fp32, o[i][j][h*32+d] bf16 (n x n)
#include "bmx_common.h"

using namespace bmx;

namespace {

constexpr int kH = 4, kD = 32, kTP = 128, kPad = 256;  // row padding: a multiple of both kTP and the attention query tile
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kProjRows = 3 * kC + 32;  // q, k, v, then H triangle-bias rows (+ zero rows)
// Triangle-bias storage type.  bf16 halves the bias traffic of the attention
// core; upstream's bf16 path rounds the bias to bf16 as well.
using tb_t = bf16;

struct Layout {
  int n, np;
  bf16 *q, *k, *vt, *o;
  tb_t* tb;
  float* mb;
};

__host__ __device__ inline int64_t qkv_elems(int np) { return (int64_t)np * kH * np * kD; }

template <typename TIn>
__device__ __forceinline__ const TIn* xrow(const TIn* x, int n, int starting, int i, int j) {
  int64_t pair = starting ? (int64_t)i * n + j : (int64_t)j * n + i;
  return x + pair * kC;
}

// ------------------------------------------------------------------ K1
template <typename TIn>
__global__ __launch_bounds__(256) void triattn_proj_kernel(const TIn* __restrict__ x, const float* __restrict__ mask,
                                                           const float* __restrict__ ln_w,
                                                           const float* __restrict__ ln_b, float eps,
                                                           const bf16* __restrict__ w_proj, float inf, int starting,
                                                           Layout L) {
  __shared__ __attribute__((aligned(16))) bf16 xt[kTP * kLdsRow];
  const int i = blockIdx.y, j0 = blockIdx.x * kTP;
  const int n = L.n, np = L.np;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6;
  auto row_ptr = [&](int p) -> const TIn* {
    int j = j0 + p;
    return (i < n && j < n) ? xrow(x, n, starting, i, j) : nullptr;
  };
  ln_rows_to_lds<kTP, TIn>(row_ptr, ln_w, ln_b, eps, xt);
  if (t < kTP) {
    int j = j0 + t;
    float mb = 0.f;
    if (i < n && j < n && mask) {
      float m = starting ? mask[(int64_t)i * n + j] : mask[(int64_t)j * n + i];
      mb = inf * (m - 1.f) * kLog2e;
    }
    L.mb[(int64_t)i * np + j] = mb;
  }
  __syncthreads();

  const float qscale = kLog2e / sqrtf((float)kD);
  // 13 weight tiles of 32 rows: 0-3 q heads, 4-7 k heads, 8-11 v heads, 12 tri-bias.
  for (int tile = w; tile < 13; tile += 4) {
    bf16x8 wf[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) wf[ks] = frag(w_proj, kC, tile * 32, ks);
    const int kind = tile >> 2, h = tile & 3;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      f32x16 acc = zero16();
      if (kind < 2) {
        // D[pair][d]: lane = d, register = pair.
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) acc = mfma32(frag(xt, kLdsRow, nt * 32, ks), wf[ks], acc);
        bf16* dst = (kind == 0 ? L.q : L.k) + (((int64_t)i * kH + h) * np + j0) * kD + (l & 31);
        const float sc = kind == 0 ? qscale : 1.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[(nt * 32 + drow(r, l)) * kD] = (bf16)(acc[r] * sc);
      } else {
        // D[channel][pair]: lane = pair, register = channel.
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) acc = mfma32(wf[ks], frag(xt, kLdsRow, nt * 32, ks), acc);
        const int j = j0 + nt * 32 + (l & 31);
        if (kind == 2) {
          bf16* dst = L.vt + ((int64_t)i * kH + h) * kD * np + j;
#pragma unroll
          for (int r = 0; r < 16; ++r) dst[(int64_t)drow(r, l) * np] = (bf16)acc[r];
        } else if (l < 32) {
#pragma unroll
          for (int r = 0; r < kH; ++r) {
            float v = j < n ? acc[r] * kLog2e : -INFINITY;
            L.tb[((int64_t)r * np + i) * np + j] = (tb_t)v;
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ K2
constexpr int kKT = 64;             // keys per pipeline stage
constexpr int kKLd = kD + 8;        // K tile row (bf16)
constexpr int kVLd = kKT + 8;       // V^T tile row (bf16)

// Rescale the running output only when a query's max grows by more than
// 2^kLazy: until then p = exp2(s - m) stays <= 2^kLazy, exact in fp32/bf16.
constexpr float kLazy = 8.f;

// Blocks are dispatched round-robin over the 8 XCDs.  A "column" is one
// (head, query tile); every XCD owns a contiguous run of columns, so the
// triangle-bias rows those columns re-read for every row i stay in that
// XCD's L2 instead of being fetched again from HBM / MALL.
constexpr int kCoreWaves = 4;              // waves per attention block
constexpr int kCoreQ = 32 * kCoreWaves;    // queries per attention block
constexpr int kCoreThreads = 64 * kCoreWaves;

__host__ __device__ inline int core_qtiles(int n) { return (n + kCoreQ - 1) / kCoreQ; }
__host__ __device__ inline int core_cols_per_xcd(int n) { return (kH * core_qtiles(n) + 7) / 8; }

// Rows i processed together by one block: every triangle-bias tile loaded
// into registers serves all of them, which divides the dominant bias
// traffic (N x the [H, N, N] bias per direction) by kRows.
constexpr int kRows = 2;

template <bool MASKED>
__device__ __forceinline__ void core_rows(const Layout& L, int i0, int h, int q0, bf16* ks, bf16* vs) {
  constexpr int G = kRows;
  constexpr int kKs = kKT * kKLd, kVs = kD * kVLd;  // per-row LDS tile sizes
  const int n = L.n, np = L.np;
  const int t = threadIdx.x, l = lane_id(), hf = l >> 5;
  const int nk = (n + kKT - 1) / kKT * kKT;
  const tb_t* tbrow = L.tb + ((int64_t)h * np + q0 + (l & 31)) * np;
  const bf16* kb[G];
  const bf16* vb[G];
  const float* mbr[G];
  bf16x8 qf[G][2];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int i = min(i0 + g, n - 1);  // rows past n repeat row n-1 and are not stored
    kb[g] = L.k + ((int64_t)i * kH + h) * np * kD;
    vb[g] = L.vt + ((int64_t)i * kH + h) * kD * np;
    mbr[g] = L.mb + (int64_t)i * np;
    const bf16* qbase = L.q + (((int64_t)i * kH + h) * np + q0) * kD;
    qf[g][0] = frag(qbase, kD, 0, 0);
    qf[g][1] = frag(qbase, kD, 0, 1);
  }
  f32x16 o[G];
  float m[G], lsum[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    o[g] = zero16();
    m[g] = -INFINITY;
    lsum[g] = 0.f;
  }
  // Per row and stage: K tile 64 keys x 32 d and V^T tile 32 d x 64 keys,
  // 256 chunks of 8 each; chunk c < 256 is K, c >= 256 is V^T.
  constexpr int kPer = 512 / kCoreThreads;
  static_assert(kPer * kCoreThreads == 512, "K/V chunks must split evenly over the block");
  bf16x8 rkv[G][kPer];
  auto gload = [&](int k0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int c = 0; c < kPer; ++c) {
        const int idx = t + kCoreThreads * c, u = idx & 255;
        rkv[g][c] = idx < 256 ? *(const bf16x8*)(kb[g] + (int64_t)(k0 + (u >> 2)) * kD + (u & 3) * 8)
                              : *(const bf16x8*)(vb[g] + (int64_t)(u >> 3) * np + k0 + (u & 7) * 8);
      }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int c = 0; c < kPer; ++c) {
        const int idx = t + kCoreThreads * c, u = idx & 255;
        bf16* dst = idx < 256 ? ks + (buf * G + g) * kKs + (u >> 2) * kKLd + (u & 3) * 8
                              : vs + (buf * G + g) * kVs + (u >> 3) * kVLd + (u & 7) * 8;
        *(bf16x8*)dst = rkv[g][c];
      }
  };
  gload(0);
  sstore(0);
  __syncthreads();
  for (int k0 = 0; k0 < nk; k0 += kKT) {
    const int cur = (k0 / kKT) & 1;
    const bool more = k0 + kKT < nk;
    // Triangle-bias C tiles for these 64 keys: lane = query, register r -> key drow(r).
    f32x16 cb[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        f32x4 v = load4(tbrow + k0 + 32 * sub + 4 * hf + 8 * gq);
#pragma unroll
        for (int e = 0; e < 4; ++e) cb[sub][4 * gq + e] = v[e];
      }
    if (more) gload(k0 + kKT);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const bf16* kt = ks + (cur * G + g) * kKs;
      f32x16 s[2];
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        f32x16 c = cb[sub];
        if (MASKED) {
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            f32x4 v = *(const f32x4*)(mbr[g] + k0 + 32 * sub + 4 * hf + 8 * gq);
#pragma unroll
            for (int e = 0; e < 4; ++e) c[4 * gq + e] += v[e];
          }
        }
        const bf16* ksub = kt + 32 * sub * kKLd;
        s[sub] = mfma32(frag(ksub, kKLd, 0, 1), qf[g][1], mfma32(frag(ksub, kKLd, 0, 0), qf[g][0], c));
      }
      float mt = s[0][0];
#pragma unroll
      for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[0][r]);
#pragma unroll
      for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[1][r]);
      mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
      if (__any(mt > m[g] + kLazy)) {  // wave-uniform; rare after the first tiles
        const float mn = fmaxf(m[g], mt);
        const float alpha = __builtin_amdgcn_exp2f(m[g] - mn);
        m[g] = mn;
        lsum[g] *= alpha;
        o[g] = o[g] * alpha;
      }
      const bf16* vt = vs + (cur * G + g) * kVs;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub)
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          bf16x8 pf;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float p = __builtin_amdgcn_exp2f(s[sub][8 * st + e] - m[g]);
            lsum[g] += p;
            pf[e] = (bf16)p;
          }
          // V^T fragment with the key order of P's D-layout registers.
          const bf16* vr = vt + (l & 31) * kVLd + 32 * sub + 16 * st + 4 * hf;
          bf16x4 v0 = *(const bf16x4*)vr, v1 = *(const bf16x4*)(vr + 8);
          bf16x8 vf = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
          o[g] = mfma32(vf, pf, o[g]);
        }
    }
    if (more) sstore(cur ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float ls = lsum[g] + __shfl_xor(lsum[g], 32, kWave);
    const int q = q0 + (l & 31);
    if (i0 + g < n && q < n) {
      const float inv = 1.f / ls;
      bf16* dst = L.o + ((int64_t)(i0 + g) * n + q) * kC + h * kD + 4 * hf;
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        bf16x4 pk = {(bf16)(o[g][4 * gq] * inv), (bf16)(o[g][4 * gq + 1] * inv), (bf16)(o[g][4 * gq + 2] * inv),
                     (bf16)(o[g][4 * gq + 3] * inv)};
        *(bf16x4*)(dst + 8 * gq) = pk;
      }
    }
  }
}

__host__ __device__ inline int core_row_groups(int n) { return (n + kRows - 1) / kRows; }

__global__ __launch_bounds__(kCoreThreads) void triattn_core_kernel(Layout L) {
  __shared__ __attribute__((aligned(16))) bf16 ks_lds[2 * kRows * kKT * kKLd];
  __shared__ __attribute__((aligned(16))) bf16 vs_lds[2 * kRows * kD * kVLd];
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
  const int q0 = qt * kCoreQ + 32 * w;  // this wave's 32 queries (< np: np is a multiple of kCoreQ)

  bool masked = false;
  for (int g = 0; g < kRows && i0 + g < n; ++g) {
    const float* mbrow = L.mb + (int64_t)(i0 + g) * np;
    for (int k = t; k < n; k += kCoreThreads) masked |= mbrow[k] != 0.f;
  }
  masked = __syncthreads_or(masked);
  if (masked)
    core_rows<true>(L, i0, h, q0, ks_lds, vs_lds);
  else
    core_rows<false>(L, i0, h, q0, ks_lds, vs_lds);
}

// ------------------------------------------------------------------ K3
// Persistent and weight-stationary; a tile is 64 positions (i, j0..j0+63) of
// the row frame.  Input rows stay in registers from the prefetch to the
// residual store, so x is read once; results are re-laid out through LDS.
constexpr int kP3 = 64;

template <typename TIn>
__global__ __launch_bounds__(256, 2) void triattn_out_kernel(const TIn* x, const float* __restrict__ ln_w,
                                                             const float* __restrict__ ln_b, float eps,
                                                             const bf16* __restrict__ w_g,
                                                             const float* __restrict__ b_g,
                                                             const bf16* __restrict__ w_o,
                                                             const float* __restrict__ b_o, int starting, void* out,
                                                             int out_mode, Layout L) {
  __shared__ __attribute__((aligned(16))) bf16 smem[2 * kP3 * kLdsRow];
  bf16* xg = smem;                   // LN(x'), pairs x channels
  bf16* xo = smem + kP3 * kLdsRow;   // attention output, then o * gate
  float* ybuf = (float*)smem;        // fp32 result rows (aliases both)
  static_assert(kP3 * kYRow * 4 <= 2 * kP3 * kLdsRow * 2, "ybuf must fit in the tile buffers");
  const int n = L.n;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6, c0 = 32 * w, ch = c0 + (l & 31);
  const int hw = t >> 5, hl = t & 31;
  const int tiles_x = (n + kP3 - 1) / kP3, total = n * tiles_x;
  const bool x_in_regs = out_mode == kOutResidual || (const void*)x == out;

  bf16x8 wg[8], wo[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) {
    wg[ks] = frag(w_g, kC, c0, ks);
    wo[ks] = frag(w_o, kC, c0, ks);
  }
  const float bg = b_g[ch], bo = b_o[ch];

  constexpr int kRowsPer = kP3 / 8;
  f32x4 px[kRowsPer];
  bf16x4 po[kRowsPer];
  auto fetch = [&](int tile) {
    const int i = tile / tiles_x, j0 = (tile % tiles_x) * kP3;
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      const int j = j0 + hw + 8 * u;
      if (j < n) {
        px[u] = load4(xrow(x, n, starting, i, j) + 4 * hl);
        po[u] = *(const bf16x4*)(L.o + ((int64_t)i * n + j) * kC + 4 * hl);
      } else {
        px[u] = f32x4{0.f, 0.f, 0.f, 0.f};
        po[u] = bf16x4{};
      }
    }
  };

  int tile = blockIdx.x;
  if (tile < total) fetch(tile);
  for (; tile < total; tile += gridDim.x) {
    const int i = tile / tiles_x, j0 = (tile % tiles_x) * kP3;
    f32x4 xc[kRowsPer];
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      xc[u] = px[u];
      f32x4 y = ln128_half(px[u], ln_w, ln_b, hl, eps);
      bf16x4 o = {(bf16)y[0], (bf16)y[1], (bf16)y[2], (bf16)y[3]};
      *(bf16x4*)(xg + (hw + 8 * u) * kLdsRow + 4 * hl) = o;
      *(bf16x4*)(xo + (hw + 8 * u) * kLdsRow + 4 * hl) = po[u];
    }
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
    f32x16 res[kP3 / 32];
#pragma unroll
    for (int nt = 0; nt < kP3 / 32; ++nt) {
      f32x16 acc = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) acc = mfma32(frag(xo, kLdsRow, nt * 32, ks), wo[ks], acc);
#pragma unroll
      for (int r = 0; r < 16; ++r) res[nt][r] = rbf(acc[r] + bo);
    }
    __syncthreads();  // xg / xo are dead; ybuf aliases them
#pragma unroll
    for (int nt = 0; nt < kP3 / 32; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) ybuf[(nt * 32 + drow(r, l)) * kYRow + ch] = res[nt][r];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < kRowsPer; ++u) {
      const int p = hw + 8 * u, j = j0 + p;
      if (j < n) {
        const f32x4 y = *(const f32x4*)(ybuf + p * kYRow + 4 * hl);
        const int64_t pair = starting ? (int64_t)i * n + j : (int64_t)j * n + i;
        store_row4(out, pair * kC + 4 * hl, y, xc[u], out_mode, x_in_regs);
      }
    }
    __syncthreads();
  }
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
  return L;
}

template <typename TIn>
int run(const TIn* x, const float* mask, int n, int starting, float inf, const float* ln_w, const float* ln_b,
        float eps, const bf16* w_proj, const bf16* w_g, const float* b_g, const bf16* w_o, const float* b_o,
        void* out, int out_mode, void* ws, int stages, hipStream_t st) {
  Layout L = make_layout(ws, n);
  if (stages & 1) {
    triattn_proj_kernel<TIn><<<dim3(L.np / kTP, L.np), 256, 0, st>>>(x, mask, ln_w, ln_b, eps, w_proj, inf,
                                                                      starting, L);
    if (int rc = check_launch("triattn_proj")) return rc;
  }
  if (stages & 2) {
    triattn_core_kernel<<<dim3((unsigned)(8ll * core_cols_per_xcd(n) * core_row_groups(n))), kCoreThreads, 0, st>>>(L);
    if (int rc = check_launch("triattn_core")) return rc;
  }
  if (stages & 4) {
    const int total = n * ((n + kP3 - 1) / kP3);
    const int grid = total < 2 * device_cu_count() ? total : 2 * device_cu_count();
    triattn_out_kernel<TIn><<<dim3(grid), 256, 0, st>>>(x, ln_w, ln_b, eps, w_g, b_g, w_o, b_o, starting, out,
                                                        out_mode, L);
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
                  np * np * 4);
}

int bmx_triattn_fwd(const void* x, int x_dtype, const float* mask, int64_t n, int starting, float inf,
                    const float* ln_w, const float* ln_b, float eps, const void* w_proj, const void* w_g,
                    const float* b_g, const void* w_o, const float* b_o, void* out, int out_mode, void* workspace,
                    size_t workspace_bytes, int stages, hipStream_t stream) {
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
                      (const bf16*)w_g, b_g, (const bf16*)w_o, b_o, out, out_mode, workspace, stages, stream);
  return run<bf16>((const bf16*)x, mask, (int)n, starting, inf, ln_w, ln_b, eps, (const bf16*)w_proj,
                   (const bf16*)w_g, b_g, (const bf16*)w_o, b_o, out, out_mode, workspace, stages, stream);
}

int bmx_triattn_proj_rows(void) { return kProjRows; }

}  // extern "C"
