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

constexpr int kH = 4, kD = 32, kTP = 128, kPad = 128;
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kProjRows = 3 * kC + 32;  // q, k, v, then H triangle-bias rows (+ zero rows)

struct Layout {
  int n, np;
  bf16 *q, *k, *vt, *o;
  float *tb, *mb;
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
            L.tb[((int64_t)r * np + i) * np + j] = v;
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

__global__ __launch_bounds__(256) void triattn_core_kernel(Layout L) {
  __shared__ __attribute__((aligned(16))) bf16 ks_lds[2][kKT * kKLd];
  __shared__ __attribute__((aligned(16))) bf16 vs_lds[2][kD * kVLd];
  const int n = L.n, np = L.np;
  const int qtiles = (n + kTP - 1) / kTP;
  const int bid = blockIdx.x;
  const int qt = bid % qtiles, h = (bid / qtiles) % kH, i = bid / (qtiles * kH);
  const int t = threadIdx.x, l = lane_id(), w = t >> 6, hf = l >> 5;
  const int q0 = qt * kTP + 32 * w;  // this wave's 32 queries
  const int nk = (n + kKT - 1) / kKT * kKT;

  const float* mbrow = L.mb + (int64_t)i * np;
  bool masked_row = false;
  for (int k = t; k < n; k += 256) masked_row |= mbrow[k] != 0.f;
  masked_row = __syncthreads_or(masked_row);

  const bf16* kbase = L.k + ((int64_t)i * kH + h) * np * kD;
  const bf16* vbase = L.vt + ((int64_t)i * kH + h) * kD * np;
  const float* tbrow = L.tb + ((int64_t)h * np + q0 + (l & 31)) * np;

  // Q^T fragments (B operand): lane = query, 8 consecutive d per k-step.
  const bf16* qbase = L.q + (((int64_t)i * kH + h) * np + q0) * kD;
  const bf16x8 qf0 = frag(qbase, kD, 0, 0), qf1 = frag(qbase, kD, 0, 1);

  bf16x8 rk, rv;
  auto gload = [&](int k0) {
    // K tile: 64 keys x 32 d -> 256 chunks of 8; V^T tile: 32 d x 64 keys.
    rk = *(const bf16x8*)(kbase + (int64_t)(k0 + (t >> 2)) * kD + (t & 3) * 8);
    rv = *(const bf16x8*)(vbase + (int64_t)(t >> 3) * np + k0 + (t & 7) * 8);
  };
  auto sstore = [&](int buf) {
    *(bf16x8*)(&ks_lds[buf][(t >> 2) * kKLd + (t & 3) * 8]) = rk;
    *(bf16x8*)(&vs_lds[buf][(t >> 3) * kVLd + (t & 7) * 8]) = rv;
  };

  f32x16 o = zero16();
  float m = -INFINITY, lsum = 0.f;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int k0 = 0; k0 < nk; k0 += kKT) {
    const int cur = (k0 / kKT) & 1;
    if (k0 + kKT < nk) gload(k0 + kKT);
    f32x16 s[2];
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      // C operand: bias^T tile, lane = query, register r -> key drow(r).
      const int kb = k0 + 32 * sub + 4 * hf;
      f32x16 c;
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        f32x4 v = *(const f32x4*)(tbrow + kb + 8 * g);
        if (masked_row) v = v + *(const f32x4*)(mbrow + kb + 8 * g);
        c[4 * g] = v[0];
        c[4 * g + 1] = v[1];
        c[4 * g + 2] = v[2];
        c[4 * g + 3] = v[3];
      }
      const bf16* kt = &ks_lds[cur][32 * sub * kKLd];
      c = mfma32(frag(kt, kKLd, 0, 0), qf0, c);
      s[sub] = mfma32(frag(kt, kKLd, 0, 1), qf1, c);
    }
    float mt = s[0][0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mt = fmaxf(mt, s[0][r]);
#pragma unroll
    for (int r = 0; r < 16; ++r) mt = fmaxf(mt, s[1][r]);
    mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
    const float mn = fmaxf(m, mt);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    m = mn;
    lsum *= alpha;
    o = o * alpha;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) {
      const bf16* vt = &vs_lds[cur][32 * sub];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        bf16x8 pf, vf;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float p = __builtin_amdgcn_exp2f(s[sub][8 * st + e] - mn);
          lsum += p;
          pf[e] = (bf16)p;
        }
        // V^T fragment with the key order of P's D-layout registers.
        const bf16* vr = vt + (l & 31) * kVLd + 16 * st + 4 * hf;
        bf16x4 v0 = *(const bf16x4*)vr, v1 = *(const bf16x4*)(vr + 8);
        vf = bf16x8{v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
        o = mfma32(vf, pf, o);
      }
    }
    if (k0 + kKT < nk) sstore(cur ^ 1);
    __syncthreads();
  }
  lsum += __shfl_xor(lsum, 32, kWave);
  const int q = q0 + (l & 31);
  if (q < n) {
    const float inv = 1.f / lsum;
    bf16* dst = L.o + ((int64_t)i * n + q) * kC + h * kD + 4 * hf;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      bf16x4 pk = {(bf16)(o[4 * g] * inv), (bf16)(o[4 * g + 1] * inv), (bf16)(o[4 * g + 2] * inv),
                   (bf16)(o[4 * g + 3] * inv)};
      *(bf16x4*)(dst + 8 * g) = pk;
    }
  }
}

// ------------------------------------------------------------------ K3
template <typename TIn>
__global__ __launch_bounds__(256) void triattn_out_kernel(const TIn* x, const float* __restrict__ ln_w,
                                                          const float* __restrict__ ln_b, float eps,
                                                          const bf16* __restrict__ w_g, const float* __restrict__ b_g,
                                                          const bf16* __restrict__ w_o, const float* __restrict__ b_o,
                                                          int starting, void* out, int out_mode, Layout L) {
  __shared__ __attribute__((aligned(16))) bf16 xg[kTP * kLdsRow];  // LN(x'), then unused
  __shared__ __attribute__((aligned(16))) bf16 xo[kTP * kLdsRow];  // attention output, then o * gate
  const int i = blockIdx.y, j0 = blockIdx.x * kTP;
  const int n = L.n;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6;
  auto row_ptr = [&](int p) -> const TIn* {
    int j = j0 + p;
    return j < n ? xrow(x, n, starting, i, j) : nullptr;
  };
  ln_rows_to_lds<kTP, TIn>(row_ptr, ln_w, ln_b, eps, xg);
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    int idx = t + 256 * u, p = idx >> 4, chunk = idx & 15;
    bf16x8 v = {};
    if (j0 + p < n) v = *(const bf16x8*)(L.o + ((int64_t)i * n + j0 + p) * kC + chunk * 8);
    *(bf16x8*)(xo + p * kLdsRow + chunk * 8) = v;
  }
  __syncthreads();

  // Gate: D[pair][ch], lane = channel c0 + l%32.
  const int c0 = 32 * w, ch = c0 + (l & 31);
  {
    bf16x8 wf[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) wf[ks] = frag(w_g, kC, c0, ks);
    const float bg = b_g[ch];
    float gv[4][16];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      f32x16 acc = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) acc = mfma32(frag(xg, kLdsRow, nt * 32, ks), wf[ks], acc);
#pragma unroll
      for (int r = 0; r < 16; ++r) gv[nt][r] = rbf(sigmoid_f(rbf(acc[r] + bg)));
    }
    // Each (pair, channel) of xo is owned by exactly one lane here.
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        bf16* e = xo + (nt * 32 + drow(r, l)) * kLdsRow + ch;
        *e = (bf16)((float)*e * gv[nt][r]);
      }
  }
  __syncthreads();
  bf16x8 wf[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) wf[ks] = frag(w_o, kC, c0, ks);
  const float bo = b_o[ch];
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    f32x16 acc = zero16();
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) acc = mfma32(frag(xo, kLdsRow, nt * 32, ks), wf[ks], acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      int j = j0 + nt * 32 + drow(r, l);
      if (j >= n) continue;
      float y = rbf(acc[r] + bo);
      int64_t pair = starting ? (int64_t)i * n + j : (int64_t)j * n + i;
      int64_t off = pair * kC + ch;
      if (out_mode == 0)
        ((bf16*)out)[off] = (bf16)y;
      else if (out_mode == 1)
        ((float*)out)[off] = y;
      else if (out_mode == 2)
        ((float*)out)[off] += y;
      else
        ((float*)out)[off] = (float)x[off] + y;
    }
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
  L.tb = (float*)p;
  p += (int64_t)kH * L.np * L.np * sizeof(float);
  L.mb = (float*)p;
  return L;
}

template <typename TIn>
int run(const TIn* x, const float* mask, int n, int starting, float inf, const float* ln_w, const float* ln_b,
        float eps, const bf16* w_proj, const bf16* w_g, const float* b_g, const bf16* w_o, const float* b_o,
        void* out, int out_mode, void* ws, int stages, hipStream_t st) {
  Layout L = make_layout(ws, n);
  const int qtiles = (n + kTP - 1) / kTP;
  if (stages & 1) {
    triattn_proj_kernel<TIn><<<dim3(L.np / kTP, L.np), 256, 0, st>>>(x, mask, ln_w, ln_b, eps, w_proj, inf,
                                                                      starting, L);
    if (int rc = check_launch("triattn_proj")) return rc;
  }
  if (stages & 2) {
    triattn_core_kernel<<<dim3((unsigned)((int64_t)n * kH * qtiles)), 256, 0, st>>>(L);
    if (int rc = check_launch("triattn_core")) return rc;
  }
  if (stages & 4) {
    triattn_out_kernel<TIn><<<dim3(qtiles, n), 256, 0, st>>>(x, ln_w, ln_b, eps, w_g, b_g, w_o, b_o, starting,
                                                             out, out_mode, L);
    if (int rc = check_launch("triattn_out")) return rc;
  }
  return BMX_OK;
}

}  // namespace

extern "C" {

size_t bmx_triattn_workspace_bytes(int64_t n) {
  if (n <= 0) return 0;
  int64_t np = round_up(n, kPad);
  return (size_t)(3 * qkv_elems((int)np) * 2 + round_up(n * n * kC * 2, 256) + (int64_t)kH * np * np * 4 +
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
