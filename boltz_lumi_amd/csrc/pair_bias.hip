// Pair bias of the Pairformer sequence stack: bias[h][pair] = Linear(LN(z[pair]))[h]
// for 16 heads, in fp32, one pass over z.
//
// Upstream AttentionPairBias.proj_z = Sequential(LayerNorm(128), Linear(128, 16,
// no bias), Rearrange("b ... h -> b h ...")) runs outside autocast in fp32 (the
// reference leaves the sequence stack unpatched, adapters.py:39-45; math as
// pair_bias.py:21-36).  Upstream spends a LayerNorm pass writing a normalised
// copy of z and a skinny GEMM re-reading it; here z is read once, normalised
// in registers, staged in LDS and projected with fp32 MFMA
// (v_mfma_f32_16x16x4f32: the 16 heads are exactly the M tile), and the result
// is written head-major so it is the [B, H, N, N] bias without a transpose.
#include "bmx_common.h"

using namespace bmx;

namespace {

constexpr int kHeads = 16;
constexpr int kTile = 64;          // pairs per block: 4 waves x 16
constexpr int kXRow = kC + 4;      // fp32 LDS row

// 16x16x4 f32 fragments (lane l, group g = l / 16): A holds A[l%16][k=g],
// B holds B[k=g][l%16], D register r holds D[4*g + r][l%16].
// Persistent: a block keeps the weights in VGPRs and walks tiles of 64 pairs
// (4 waves x 16), prefetching the next tile's rows into registers while the
// current tile is normalised and projected.
template <typename TIn>
__global__ __launch_bounds__(256) void pair_bias_kernel(const TIn* __restrict__ z, const float* __restrict__ ln_w,
                                                        const float* __restrict__ ln_b, float eps,
                                                        const float* __restrict__ w, float* __restrict__ out,
                                                        int64_t rows) {
  __shared__ __attribute__((aligned(16))) float xs[kTile * kXRow];
  const int t = threadIdx.x, l = lane_id(), wv = t >> 6, g = l >> 4;
  const int hw = t >> 5, hl = t & 31;
  const LnAffine aff = ln_affine(ln_w, ln_b, hl);
  const int64_t tiles = (rows + kTile - 1) / kTile;

  // Weight fragments: head l%16, k = 4*s + g for the 32 k-steps.
  float wa[kC / 4];
#pragma unroll
  for (int s = 0; s < kC / 4; ++s) wa[s] = w[(l & 15) * kC + 4 * s + g];

  // Rows past the end re-read the last row (unconditional loads) and are not stored.
  f32x4 v[kTile / 8];
  auto fetch = [&](int64_t tile) {
#pragma unroll
    for (int u = 0; u < kTile / 8; ++u) v[u] = load4(z + min(tile * kTile + hw + 8 * u, rows - 1) * kC + 4 * hl);
  };
  int64_t tile = blockIdx.x;
  if (tile < tiles) fetch(tile);
  for (; tile < tiles; tile += gridDim.x) {
#pragma unroll
    for (int u = 0; u < kTile / 8; ++u) *(f32x4*)(xs + (hw + 8 * u) * kXRow + 4 * hl) = ln128_half(v[u], aff, eps);
    __syncthreads();
    if (tile + gridDim.x < tiles) fetch(tile + gridDim.x);

    // D[head][pair] = W[head][k] * X^T[k][pair]; wave wv owns pairs 16*wv .. +15.
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const float* xrow = xs + (16 * wv + (l & 15)) * kXRow + g;
#pragma unroll
    for (int s = 0; s < kC / 4; ++s) acc = mfma16f32(wa[s], xrow[4 * s], acc);
    const int64_t pair = tile * kTile + 16 * wv + (l & 15);
    if (pair < rows) {
#pragma unroll
      for (int r = 0; r < 4; ++r) out[(int64_t)(4 * g + r) * rows + pair] = acc[r];
    }
    __syncthreads();
  }
}

// ------------------------------------------------------------------
// Pair-biased attention of AttentionPairBias, fp32, one pass:
//   out[i][h*D+d] = sigmoid(g[i][h*D+d]) * sum_j softmax_j(q_i.k_j / sqrt(D) + bias[h][i][j]
//                                                          + (1 - mask[j]) * -inf) v_j[d]
// for D = 24 (Pairformer sequence stack, 16 x 24) or 48 (diffusion token
// transformer, 16 x 48); upstream AttentionPairBias, math as
// pair_bias.py:21-36; the [H, N, N] logits never reach HBM.
//
// Both products run on fp32 MFMA (v_mfma_f32_16x16x4f32; lane l, group
// gi = l / 16: A holds A[l%16][k = gi], B holds B[k = gi][l%16], D register r
// holds D[4 gi + r][l%16]).  A block owns 16 queries of one head; its 4 waves
// split the keys (wave w takes the 64-key steps w, w + 4, ...) and merge
// their softmax states through LDS at the end.  Per 16-key tile:
//   S[key][q]   = K Q^T        A = K rows, B = Q^T; the D head dims are the
//                              k index (D/4) gi + s of D/4 MFMA steps;
//   O^T[d][q]  += V^T P^T      B = P^T is the S tile itself (register s of
//                              lane (q, gi) is key 4 gi + s, the k index of
//                              step s), A = V^T in ceil(D/16) 16-row d tiles
//                              (rows past D are zero).
// Every lane then holds whole columns (one query) of S and O^T, so the
// running max and the rescale need only the xor-16 / xor-32 exchanges.
constexpr int kAttnQ = 16, kAttnWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;

// Batched shapes: element b of grid.z attends its nq query rows (q, g at row
// stride ldq, element stride sq) over its nk key rows (k, v at ldk, sk) with
// bias element b / bdiv ([heads][nq][nk], element stride sbias; upstream
// repeat_interleave(multiplicity)) and mask element b (stride smask, 0 to
// broadcast one mask); out element b is [nq][heads * D] at stride nq * heads * D.
struct SeqAttnShape {
  int nq, nk, bdiv;
  int64_t ldq, ldk, sq, sk, sbias, smask;
};

// TILES 16-key tiles per wave and step: 4 (64 keys), or 2 for short key rows
// (the atom transformer's 128 keys), so that all four waves get keys.
template <int D, int TILES>
__global__ __launch_bounds__(256) void seq_attention_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v,
                                                            const float* __restrict__ bias,
                                                            const float* __restrict__ mask,
                                                            const float* __restrict__ g, SeqAttnShape sh, int heads,
                                                            float inf, float rscale, bool vec,
                                                            float* __restrict__ out) {
  constexpr int KS = D / 4;          // QK^T MFMA steps
  constexpr int DT = (D + 15) / 16;  // O^T d tiles
  static_assert(D % 4 == 0, "head dim");
  const int HD = heads * D;
  const int nq = sh.nq, nk = sh.nk;
  const int64_t ldq = sh.ldq, ldk = sh.ldk;
  {
    const int64_t b = blockIdx.z;
    q += b * sh.sq;
    g += b * sh.sq;
    k += b * sh.sk;
    v += b * sh.sk;
    bias += (b / sh.bdiv) * sh.sbias;
    mask += b * sh.smask;
    out += b * nq * HD;
  }
  __shared__ float part_o[kAttnWaves][16 * DT][kAttnQ];
  __shared__ float part_m[kAttnWaves][kAttnQ], part_l[kAttnWaves][kAttnQ];
  const int h = blockIdx.y, q0 = blockIdx.x * kAttnQ;
  const int w = threadIdx.x >> 6, l = lane_id(), gi = l >> 4, c = l & 15;
  const int qc = min(q0 + c, nq - 1);  // rows past the end re-read the last one and are not stored
  float qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qf[s] = q[(int64_t)qc * ldq + h * D + KS * gi + s];
  const float* brow = bias + ((int64_t)h * nq + qc) * nk;
  f32x4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -3.4e38f, lsum = 0.f;
  constexpr int kStep = 16 * TILES;
  for (int key0 = w * kStep; key0 < nk; key0 += kAttnWaves * kStep) {
    const bool full = vec && key0 + kStep <= nk;
    f32x4 st[TILES];
    float tmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const int kr = min(key0 + 16 * t + c, nk - 1);
      const float* krow = k + (int64_t)kr * ldk + h * D + KS * gi;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = mfma16f32(krow[s], qf[s], acc);
      const int kb = key0 + 16 * t + 4 * gi;  // this lane's keys kb .. kb + 3
      f32x4 b4, m4;
      if (full) {
        b4 = *(const f32x4*)(brow + kb);
        m4 = *(const f32x4*)(mask + kb);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          b4[r] = brow[min(kb + r, nk - 1)];
          m4[r] = mask[min(kb + r, nk - 1)];
        }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float x = (acc[r] * rscale + b4[r]) + (1.f - m4[r]) * -inf;
        st[t][r] = kb + r < nk ? x : -INFINITY;
        tmax = fmaxf(tmax, st[t][r]);
      }
    }
    const float mn = fmaxf(m, col_max(tmax));
    const float alpha = __builtin_amdgcn_exp2f((m - mn) * kLog2e);
    m = mn;
    lsum *= alpha;
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] *= alpha;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const float p = __builtin_amdgcn_exp2f((st[t][s] - mn) * kLog2e);
        lsum += p;
        const int kr = min(key0 + 16 * t + 4 * gi + s, nk - 1);
        const float* vrow = v + (int64_t)kr * ldk + h * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int d = 16 * dt + c;
          const float a = vrow[d < D ? d : D - 1];  // clamped load, zero row past D
          o[dt] = mfma16f32(d < D ? a : 0.f, p, o[dt]);
        }
      }
    }
  }
  // This wave's state for its 16 queries: O^T rows 16 dt + 4 gi + r, the max
  // m, and the key sum over the four lane groups.
  lsum = col_sum(lsum);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) part_o[w][16 * dt + 4 * gi + r][c] = o[dt][r];
  if (gi == 0) part_m[w][c] = m, part_l[w][c] = lsum;
  __syncthreads();
  // Merge: thread (query qi, dim group) finishes D / 16 dims per 16 threads.
  const int qi = threadIdx.x & 15, i = q0 + qi;
  if (i < nq) {
    float mm = part_m[0][qi];
#pragma unroll
    for (int u = 1; u < kAttnWaves; ++u) mm = fmaxf(mm, part_m[u][qi]);
    float wt[kAttnWaves], ll = 0.f;
#pragma unroll
    for (int u = 0; u < kAttnWaves; ++u) {
      wt[u] = __builtin_amdgcn_exp2f((part_m[u][qi] - mm) * kLog2e);
      ll += wt[u] * part_l[u][qi];
    }
    for (int d = threadIdx.x >> 4; d < D; d += 16) {
      float acc = 0.f;
#pragma unroll
      for (int u = 0; u < kAttnWaves; ++u) acc += wt[u] * part_o[u][d][qi];
      const float gate = sigmoid_f(g[(int64_t)i * ldq + h * D + d]);
      out[(int64_t)i * HD + h * D + d] = gate * (acc / ll);
    }
  }
}

int launch_seq_attention(const char* name, const float* q, const float* k, const float* v, const float* bias,
                         const float* mask, const float* g, int64_t batch, const SeqAttnShape& sh, int heads,
                         int head_dim, float inf, float* out, hipStream_t stream) {
  // 16-byte bias / mask loads where every row start is aligned; scalar loads otherwise
  const bool vec = sh.nk % 4 == 0 && sh.sbias % 4 == 0 && sh.smask % 4 == 0 && (uintptr_t)bias % 16 == 0 &&
                   (uintptr_t)mask % 16 == 0;
  const dim3 grid((unsigned)((sh.nq + kAttnQ - 1) / kAttnQ), (unsigned)heads, (unsigned)batch);
  const float rscale = 1.f / sqrtf((float)head_dim);
#define SEQ_ATTN(DIM, TILES) \
  seq_attention_kernel<DIM, TILES><<<grid, 256, 0, stream>>>(q, k, v, bias, mask, g, sh, heads, inf, rscale, vec, out)
  const bool short_keys = sh.nk <= kAttnWaves * 32;
  if (head_dim == 24) SEQ_ATTN(24, 4);
  else if (head_dim == 32 && short_keys) SEQ_ATTN(32, 2);
  else if (head_dim == 32) SEQ_ATTN(32, 4);
  else SEQ_ATTN(48, 4);
#undef SEQ_ATTN
  return check_launch(name);
}

}  // namespace

extern "C" {

int bmx_pair_bias_fwd(const void* z, int z_dtype, int64_t rows, const float* ln_w, const float* ln_b, float eps,
                      const float* w, int heads, float* out, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0, "bmx_pair_bias_fwd: rows must be >= 0");
  BMX_REQUIRE(heads == kHeads, "bmx_pair_bias_fwd: built for %d heads (got %d)", kHeads, heads);
  BMX_REQUIRE(z_dtype == kF32 || z_dtype == kBF16, "bmx_pair_bias_fwd: z dtype must be fp32 or bf16");
  BMX_REQUIRE(eps > 0.f, "bmx_pair_bias_fwd: eps must be positive");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(z && ln_w && ln_b && w && out, "bmx_pair_bias_fwd: null pointer");
  BMX_REQUIRE((uintptr_t)z % 16 == 0, "bmx_pair_bias_fwd: z must be 16-byte aligned");
  const int64_t tiles = (rows + kTile - 1) / kTile;
  const unsigned grid = (unsigned)(tiles < 4 * device_cu_count() ? tiles : 4 * device_cu_count());
  if (z_dtype == kF32)
    pair_bias_kernel<float><<<grid, 256, 0, stream>>>((const float*)z, ln_w, ln_b, eps, w, out, rows);
  else
    pair_bias_kernel<bf16><<<grid, 256, 0, stream>>>((const bf16*)z, ln_w, ln_b, eps, w, out, rows);
  return check_launch("bmx_pair_bias_fwd");
}

int bmx_seq_attention_fwd(const float* q, const float* k, const float* v, const float* bias, const float* mask,
                          const float* g, int64_t n, int64_t ld, int heads, int head_dim, float inf, float* out,
                          hipStream_t stream) {
  BMX_REQUIRE(n >= 0 && n <= (1 << 20), "bmx_seq_attention_fwd: n must be in [0, 2^20]");
  BMX_REQUIRE(head_dim == 24 || head_dim == 48, "bmx_seq_attention_fwd: head_dim must be 24 or 48 (got %d)", head_dim);
  BMX_REQUIRE(heads >= 1 && heads <= 64, "bmx_seq_attention_fwd: heads must be in [1, 64] (got %d)", heads);
  BMX_REQUIRE(ld >= (int64_t)heads * head_dim, "bmx_seq_attention_fwd: row stride ld must be >= heads * head_dim");
  BMX_REQUIRE(inf > 0.f, "bmx_seq_attention_fwd: inf must be positive");
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(q && k && v && bias && mask && g && out, "bmx_seq_attention_fwd: null pointer");
  const SeqAttnShape sh{(int)n, (int)n, 1, ld, ld, 0, 0, 0, 0};
  return launch_seq_attention("bmx_seq_attention_fwd", q, k, v, bias, mask, g, 1, sh, heads, head_dim, inf, out,
                              stream);
}

int bmx_seq_attention_batched_fwd(const float* q, const float* k, const float* v, const float* bias,
                                  const float* mask, const float* g, int64_t batch, int64_t nq, int64_t nk,
                                  int64_t ldq, int64_t ldk, int64_t sq, int64_t sk, int64_t sbias, int64_t smask,
                                  int64_t bias_div, int heads, int head_dim, float inf, float* out,
                                  hipStream_t stream) {
  BMX_REQUIRE(batch >= 0 && batch <= 65535, "bmx_seq_attention_batched_fwd: batch must be in [0, 65535]");
  BMX_REQUIRE(nq >= 0 && nq <= (1 << 20) && nk >= 1 && nk <= (1 << 20),
              "bmx_seq_attention_batched_fwd: need 0 <= nq <= 2^20 and 1 <= nk <= 2^20");
  BMX_REQUIRE(head_dim == 24 || head_dim == 32 || head_dim == 48,
              "bmx_seq_attention_batched_fwd: head_dim must be 24, 32 or 48 (got %d)", head_dim);
  BMX_REQUIRE(heads >= 1 && heads <= 64, "bmx_seq_attention_batched_fwd: heads must be in [1, 64] (got %d)", heads);
  BMX_REQUIRE(ldq >= (int64_t)heads * head_dim && ldk >= (int64_t)heads * head_dim,
              "bmx_seq_attention_batched_fwd: row strides must be >= heads * head_dim");
  BMX_REQUIRE(sq >= 0 && sk >= 0 && sbias >= 0 && smask >= 0 && bias_div >= 1,
              "bmx_seq_attention_batched_fwd: strides must be >= 0 and bias_div >= 1");
  BMX_REQUIRE(inf > 0.f, "bmx_seq_attention_batched_fwd: inf must be positive");
  if (batch == 0 || nq == 0) return BMX_OK;
  BMX_REQUIRE(q && k && v && bias && mask && g && out, "bmx_seq_attention_batched_fwd: null pointer");
  const SeqAttnShape sh{(int)nq, (int)nk, (int)bias_div, ldq, ldk, sq, sk, sbias, smask};
  return launch_seq_attention("bmx_seq_attention_batched_fwd", q, k, v, bias, mask, g, batch, sh, heads, head_dim,
                              inf, out, stream);
}

}  // extern "C"
