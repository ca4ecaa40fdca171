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
//
// The fp32 kernel also takes (defaults give the form above):
//  * bias element of b at (b / bdiv) * sbg + (b % bwin) * sbias (sbg < 0:
//    bwin * sbias, so element (b / bdiv) * bwin + b % bwin), with head / query
//    / key strides sbh, sbq, sbk (sbq == 0: dense [heads][nq][nk]);
//  * windowed keys (nw > 0; the atom transformer's to_keys gather): element b
//    is window b % nw of its sample, and its key j is row koff + j of its k / v
//    / mask block (sk = wq * ldk, smask = wq), present only while
//    0 <= (b % nw) * wq + koff + j < nw * wq; an absent key is a zero key and
//    value row with mask 0, as upstream's zero rows of single_to_keys.
struct SeqAttnShape {
  int nq, nk, bdiv;
  int64_t ldq, ldk, sq, sk, sbias, smask;
  int bwin = 1;
  int64_t sbh = 0, sbq = 0, sbk = 1, sbg = -1;
  int nw = 0, wq = 0, koff = 0;
};

// TILES 16-key tiles per wave and step: 4 (64 keys), or 2 for short key rows
// (the atom transformer's 128 keys), so that all four waves get keys.
template <int D, int TILES>
__global__ __launch_bounds__(256) void seq_attention_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                            const float* __restrict__ v,
                                                            const float* __restrict__ bias,
                                                            const float* __restrict__ mask,
                                                            const float* __restrict__ g, SeqAttnShape sh, int heads,
                                                            float inf, float rscale, int vec,
                                                            float* __restrict__ out) {
  constexpr int KS = D / 4;          // QK^T MFMA steps
  constexpr int DT = (D + 15) / 16;  // O^T d tiles
  static_assert(D % 4 == 0, "head dim");
  const int HD = heads * D;
  const int nq = sh.nq, nk = sh.nk;
  const int64_t ldq = sh.ldq, ldk = sh.ldk;
  int klo = 0, khi = nk;  // keys present: klo <= j < khi
  {
    const int64_t b = blockIdx.z;
    q += b * sh.sq;
    g += b * sh.sq;
    k += b * sh.sk;
    v += b * sh.sk;
    bias += (b / sh.bdiv) * sh.sbg + (b % sh.bwin) * sh.sbias;
    mask += b * sh.smask;
    out += b * nq * HD;
    if (sh.nw > 0) {
      const int t0 = (int)(b % sh.nw) * sh.wq + sh.koff;
      klo = max(0, -t0);
      khi = min(nk, sh.nw * sh.wq - t0);
      k += (int64_t)sh.koff * ldk;
      v += (int64_t)sh.koff * ldk;
      mask += sh.koff;
    }
  }
  __shared__ float part_o[kAttnWaves][16 * DT][kAttnQ];
  __shared__ float part_m[kAttnWaves][kAttnQ], part_l[kAttnWaves][kAttnQ];
  const int h = blockIdx.y, q0 = blockIdx.x * kAttnQ;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = lane_id(), gi = l >> 4, c = l & 15;
  const int qc = min(q0 + c, nq - 1);  // rows past the end re-read the last one and are not stored
  float qf[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qf[s] = q[(int64_t)qc * ldq + h * D + KS * gi + s];
  const float* brow = bias + h * sh.sbh + qc * sh.sbq;
  f32x4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -3.4e38f, lsum = 0.f;
  constexpr int kStep = 16 * TILES;
  for (int key0 = w * kStep; key0 < nk; key0 += kAttnWaves * kStep) {
    f32x4 st[TILES];
    float tmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      // 16-byte bias / mask loads for a tile whose 16 keys all exist (and, for
      // the mask, are all present)
      const int t0 = key0 + 16 * t;
      const bool bfull = (vec & 1) && t0 + 16 <= nk;
      const bool mfull = (vec & 2) && t0 >= klo && t0 + 16 <= khi;
      const int kj = key0 + 16 * t + c;
      const bool kin = kj >= klo && kj < khi;
      const float* krow = k + (int64_t)min(max(kj, klo), khi - 1) * ldk + h * D + KS * gi;
      float kv[KS];  // loaded unconditionally (the row is clamped in range), then selected
#pragma unroll
      for (int s = 0; s < KS; ++s) kv[s] = krow[s];
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) acc = mfma16f32(kin ? kv[s] : 0.f, qf[s], acc);
      const int kb = key0 + 16 * t + 4 * gi;  // this lane's keys kb .. kb + 3
      f32x4 b4, m4;
      if (bfull) {
        b4 = *(const f32x4*)(brow + kb);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) b4[r] = brow[(int64_t)min(kb + r, nk - 1) * sh.sbk];
      }
      if (mfull) {
        m4 = *(const f32x4*)(mask + kb);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int j = kb + r;
          const float mj = mask[min(max(j, klo), khi - 1)];
          m4[r] = j >= klo && j < khi ? mj : 0.f;
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
        const int kj = key0 + 16 * t + 4 * gi + s;
        const bool kin = kj >= klo && kj < khi;
        const float* vrow = v + (int64_t)min(max(kj, klo), khi - 1) * ldk + h * D;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int d = 16 * dt + c;
          const float a = vrow[d < D ? d : D - 1];  // clamped load; zero past D and for absent keys
          o[dt] = mfma16f32(d < D && kin ? a : 0.f, p, o[dt]);
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
                         const float* mask, const float* g, int64_t batch, SeqAttnShape sh, int heads,
                         int head_dim, float inf, float* out, hipStream_t stream) {
  if (sh.sbq == 0) {  // dense [heads][nq][nk] bias elements
    sh.sbh = (int64_t)sh.nq * sh.nk;
    sh.sbq = sh.nk;
    sh.sbk = 1;
  }
  if (sh.sbg < 0) sh.sbg = sh.sbias * sh.bwin;
  // 16-byte bias (bit 0) / mask (bit 1) loads where every row start is
  // aligned; scalar loads otherwise
  const int vec = (sh.sbk == 1 && sh.nk % 4 == 0 && sh.sbias % 4 == 0 && sh.sbg % 4 == 0 && sh.sbh % 4 == 0 &&
                   sh.sbq % 4 == 0 && (uintptr_t)bias % 16 == 0 ? 1 : 0) |
                  (sh.smask % 4 == 0 && sh.koff % 4 == 0 && (uintptr_t)mask % 16 == 0 ? 2 : 0);
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

// ------------------------------------------------------------------
// The same attention on bf16 MFMA with both products split into bf16 high
// and low parts (x y ~ xh yh + xh yl + xl yh, about 2^-16 relative per
// product, the form the fp32 linears of the diffusion blocks use), for long
// key rows (the token transformer's).
//
// A pre-pass writes K as bf16 hi / lo [b][h][key][d] and V^T as hi / lo
// [b][h][d][key'], keys padded with zeros to a multiple of 64 and, in V^T, permuted inside each 32-key block into the order in which a
// lane holds P: slot 8 gi + e of a block holds key 4 gi + e (e < 4) or
// 16 + 4 gi + e - 4; and each key's additive mask term (1 - mask) * -inf as
// fp32 [b][key'], -infinity past nk, so that a logit is (q.k / sqrt(D) +
// bias) + term with no per-key select.  A block serves 64 queries of one head (16 per wave) and
// walks the keys in KS-key stages (32 keys for D = 48, else 64) that LDS DMA
// copies into a double-buffered LDS
// stage shared by the four waves (K tiles dense, V^T rows of KS slots with
// their 16-byte chunks XOR-swizzled by d mod KS / 8), so each K / V element is
// read from L2 once per 64 queries.  At D = 48, 32-key stages halve the LDS of
// a block (24 KB), so 5 blocks share a CU instead of 3.  v_mfma_f32_16x16x32_bf16 (lane l, gi = l / 16:
// A holds A[l%16][8 gi .. 8 gi + 7], B holds B[8 gi .. 8 gi + 7][l%16], D
// register r holds D[4 gi + r][l%16]); per stage and wave:
//   S^T[key][q] = K Q^T         KS / 16 16-key tiles, k steps of 32 dims (a last
//                               step of 16 dims on v_mfma_f32_16x16x16_bf16 for
//                               D = 48; dims past D are zero), 3 terms;
//   O^T[d][q] += V^T P^T        KS / 32 32-key k steps per 16-dim tile, 3 terms,
//                               P^T from the lane's probabilities.
constexpr int kX3Stage = 64;  // key padding of the pre-pass, and the LDS stage where 32 keys are not whole KB
constexpr int kX3Q = 64;      // queries per block

__host__ __device__ inline int64_t x3_nkp(int64_t nk) { return (nk + kX3Stage - 1) / kX3Stage * kX3Stage; }

__device__ __forceinline__ int x3_slot(int key_in_block) {
  return ((key_in_block & 15) >> 2) * 8 + (key_in_block >> 4) * 4 + (key_in_block & 3);
}

// Block (channels span bx .., KG 32-key blocks from KG by, element b), span =
// 256 / KG: KG = 2 where the row has at most 128 channels, so that every
// thread has work.  V: thread t splits V[b][key][c] of the 32 keys of key
// block KG by + t / span, channel c = span bx + t % span, into one V^T row
// segment (four 16-byte stores).  K: each thread takes 8 consecutive channels
// of 4 of the block's keys (KG x 32 keys x span channels = 1024 such chunks),
// so a K row is read and its hi / lo rows written 16 bytes at a time (8 | D
// keeps a chunk inside one head).  VEC: K rows 16-byte aligned (element loads
// otherwise).  Keys past nk are zeros.
template <bool VEC, int KG>
__global__ __launch_bounds__(256) void seq_attn_split_kernel(const float* __restrict__ k, const float* __restrict__ v,
                                                             int nk, int64_t ldk, int64_t sk, int heads, int d,
                                                             const float* __restrict__ mask, int64_t smask, float inf,
                                                             bf16* __restrict__ kh, bf16* __restrict__ kl,
                                                             bf16* __restrict__ vth, bf16* __restrict__ vtl,
                                                             float* __restrict__ mterm) {
  constexpr int span = 256 / KG, c8 = span / 8;
  const int hd = heads * d;
  const int64_t b = blockIdx.z, nkp = x3_nkp(nk);
  if (blockIdx.x == 0 && threadIdx.x < 32 * KG) {  // the additive mask term of each key; -inf past nk
    const int key = blockIdx.y * 32 * KG + threadIdx.x;
    mterm[b * nkp + key] = key < nk ? (1.f - mask[b * smask + key]) * -inf : -INFINITY;
  }
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int chunk = threadIdx.x + 256 * it, sub = chunk / (32 * c8), rem = chunk % (32 * c8);
    const int key = (blockIdx.y * KG + sub) * 32 + rem / c8;
    const int c0 = blockIdx.x * span + 8 * (rem % c8);
    if (c0 < hd) {
      f32x4 x0 = {0.f, 0.f, 0.f, 0.f}, x1 = x0;
      if (key < nk) {
        const float* src = k + b * sk + (int64_t)key * ldk + c0;
        if (VEC) {
          x0 = *(const f32x4*)src;
          x1 = *(const f32x4*)(src + 4);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x0[e] = src[e];
            x1[e] = src[4 + e];
          }
        }
      }
      bf16x8 hi, lo;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        hi[e] = (bf16)x0[e];
        lo[e] = (bf16)(x0[e] - (float)hi[e]);
        hi[4 + e] = (bf16)x1[e];
        lo[4 + e] = (bf16)(x1[e] - (float)hi[4 + e]);
      }
      const int64_t dst = ((b * heads + c0 / d) * nkp + key) * d + c0 % d;
      *(bf16x8*)(kh + dst) = hi;
      *(bf16x8*)(kl + dst) = lo;
    }
  }
  const int c = blockIdx.x * span + threadIdx.x % span, kb = blockIdx.y * KG + threadIdx.x / span;
  if (c >= hd) return;
  const int hh = c / d, dd = c % d;
  const float* vb_src = v + b * sk + c;
  bf16x8 vh[4], vlo[4];
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    const int key = kb * 32 + e;
    const float vv = key < nk ? vb_src[(int64_t)key * ldk] : 0.f;
    const int slot = x3_slot(e);
    const bf16 vhi = (bf16)vv;
    vh[slot >> 3][slot & 7] = vhi;
    vlo[slot >> 3][slot & 7] = (bf16)(vv - (float)vhi);
  }
  const int64_t row = ((b * heads + hh) * d + dd) * nkp + kb * 32;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    *(bf16x8*)(vth + row + 8 * u) = vh[u];
    *(bf16x8*)(vtl + row + 8 * u) = vlo[u];
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ f32x4 mfma16bf_k16(bf16x4 a, bf16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c, 0,
                                                   0, 0);
}
__device__ __forceinline__ f32x4 mfma16bf(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// One LDS DMA: 64 lanes x 16 bytes from per-lane global addresses to
// lds_addr + 16 * lane; waited for explicitly (s_waitcnt vmcnt(0)) before the
// barrier that publishes the stage.
// The DMA reads M0, which the compiler writes with an SALU instruction right
// before the asm; gfx9 needs one wait state between the two (s_nop 0), which
// the compiler's hazard recognizer inserts for its own LDS DMA but cannot see
// inside inline asm: without it the DMA may use the previous M0 and write its
// 1 KB over another stage region.
__device__ __forceinline__ void lds_dma16(const void* src, unsigned lds_addr) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(lds_addr) : "memory");
}
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

template <int D>
__global__ __launch_bounds__(256) void seq_attention_x3_kernel(const float* __restrict__ q,
                                                               const bf16* __restrict__ kh, const bf16* __restrict__ kl,
                                                               const bf16* __restrict__ vth,
                                                               const bf16* __restrict__ vtl,
                                                               const float* __restrict__ mterm,
                                                               const float* __restrict__ bias,
                                                               const float* __restrict__ g, SeqAttnShape sh, int heads,
                                                               int64_t batch, float rscale, bool vec,
                                                               float* __restrict__ out, bf16* __restrict__ op) {
  constexpr bool T16 = D % 32 == 16;             // the last 16 dims on a K = 16 MFMA
  constexpr int DK = T16 ? D / 32 : (D + 31) / 32;  // QK^T k steps of 32 dims
  constexpr int DT = (D + 15) / 16;              // O^T d tiles
  // keys per LDS stage: 32 where a double-buffered 64-key stage (2 x 4 tiles x 64 x D x 2 bytes)
  // would exceed 40 KB, i.e. leave fewer than 4 blocks per CU (D = 48: 3 -> 5 blocks); 64 otherwise, where
  // the shorter stages' extra barriers cost more than the occupancy gains (D = 32: 6.29 -> 6.64 ms)
  constexpr int KS = 2 * 4 * 64 * D * 2 > 40 * 1024 ? 32 : kX3Stage;
  static_assert(KS == kX3Stage || (32 * D * 2) % 1024 == 0, "32-key tiles must be whole KB");
  constexpr int kSwz = KS / 8 - 1;               // V^T chunk swizzle mask
  constexpr int kTile = KS * D * 2;              // bytes of one K (or V^T) tile, hi or lo
  constexpr int kStage = 4 * kTile;              // K hi, K lo, V^T hi, V^T lo
  constexpr int kDmaPerWave = kStage / 1024 / kAttnWaves;
  static_assert(D % 8 == 0 && kTile % 1024 == 0 && kDmaPerWave * kAttnWaves * 1024 == kStage, "stage layout");
  __shared__ __attribute__((aligned(16))) char lds[2 * kStage];
  const int HD = heads * D;
  const int nq = sh.nq, nk = sh.nk;
  const int64_t ldq = sh.ldq, nkp = x3_nkp(nk);
  // Blocks are dispatched round-robin over the 8 XCDs (block L on XCD L % 8).
  // Work item p = (L % 8) * per_xcd + L / 8 runs in the order (bias element,
  // head, query block, element sharing the bias): the bdiv elements that read
  // one bias tile follow each other on one XCD, which fetches the tile into
  // its L2 once instead of once per element.
  const int qblocks = (nq + kX3Q - 1) / kX3Q;
  const int64_t groups = (batch + sh.bdiv - 1) / sh.bdiv;
  const int64_t per_xcd = (groups * sh.bdiv * heads * qblocks + 7) / 8;
  const int64_t p = (int64_t)(blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
  const int64_t rest = p / sh.bdiv;
  const int64_t b = rest / ((int64_t)qblocks * heads) * sh.bdiv + p % sh.bdiv;
  if (b >= batch) return;  // the padding of the last XCD's run (whole block)
  const int h = (int)((rest / qblocks) % heads), qb = (int)(rest % qblocks);
  q += b * sh.sq;
  g += b * sh.sq;
  bias += (b / sh.bdiv) * sh.sbias;
  mterm += b * nkp;
  if (out) out += b * nq * HD;
  const bf16* k_src[2] = {kh + (b * heads + h) * nkp * D, kl + (b * heads + h) * nkp * D};
  const bf16* v_src[2] = {vth + (b * heads + h) * D * nkp, vtl + (b * heads + h) * D * nkp};
  const int l = lane_id(), gi = l >> 4, c = l & 15, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int qw = qb * kX3Q + 16 * w;             // this wave's 16 queries
  const int qc = min(qw + c, nq - 1);            // rows past the end re-read the last one and are not stored
  const unsigned lds0 = (unsigned)(uintptr_t)(__attribute__((address_space(3))) void*)lds;

  // DMA job u of this wave copies stage bytes [1024 j, 1024 j + 1024), j = w + 4 u:
  // region j / (kTile / 1024) is K hi, K lo, V^T hi or V^T lo.  K tiles are
  // the dense rows of KS keys; a V^T row is KS slots (2 KS bytes) whose chunk
  // at position p holds the global chunk p ^ (d & kSwz).
  const bf16* dma_src[kDmaPerWave];
  int dma_step[kDmaPerWave];
#pragma unroll
  for (int u = 0; u < kDmaPerWave; ++u) {
    const int j = w + kAttnWaves * u, region = j / (kTile / 1024);
    const int off = (j - region * (kTile / 1024)) * 1024 + 16 * l;  // byte offset inside the tile
    if (region < 2) {
      dma_src[u] = k_src[region] + off / 2;
      dma_step[u] = KS * D;
    } else {
      const int d = off / (KS * 2), p = (off % (KS * 2)) / 16;
      dma_src[u] = v_src[region - 2] + (int64_t)d * nkp + 8 * (p ^ (d & kSwz));
      dma_step[u] = KS;
    }
  }
  auto dma_stage = [&](int buf) {
#pragma unroll
    for (int u = 0; u < kDmaPerWave; ++u) {
      const int j = w + kAttnWaves * u;
      lds_dma16(dma_src[u], __builtin_amdgcn_readfirstlane(lds0 + buf * kStage + 1024 * j));
      dma_src[u] += dma_step[u];
    }
  };

  // Q^T (B operand): dims 32 ks + 8 gi .. + 7 of query qc, split; dims past D are zero.
  bf16x8 qh[DK], ql[DK];
#pragma unroll
  for (int ks = 0; ks < DK; ++ks) {
    const int d0 = 32 * ks + 8 * gi;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float x = d0 < D ? q[(int64_t)qc * ldq + h * D + d0 + e] : 0.f;
      qh[ks][e] = (bf16)x;
      ql[ks][e] = (bf16)(x - (float)qh[ks][e]);
    }
  }
  bf16x4 qh4, ql4;  // dims 32 DK + 4 gi .. + 3 (T16)
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float x = T16 ? q[(int64_t)qc * ldq + h * D + 32 * DK + 4 * gi + e] : 0.f;
    qh4[e] = (bf16)x;
    ql4[e] = (bf16)(x - (float)qh4[e]);
  }
  const float* brow = bias + ((int64_t)h * nq + qc) * nk;
  const bf16x8 zero8 = {};
  f32x4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -3.4e38f, lsum = 0.f;
  const int nst = (int)(nkp / KS);
  // the q loads must land before the first DMA: a wait the compiler places for
  // them inside the loop would be vmcnt(0), which also waits for a DMA in flight
  wait_vm0();
  dma_stage(0);
  wait_vm0();
  __syncthreads();
  for (int st = 0; st < nst; ++st) {
    if (st + 1 < nst) dma_stage((st + 1) & 1);
    const char* sb = lds + (st & 1) * kStage;
    const int key0 = st * KS;
    const bool full = vec && key0 + KS <= nk;
    f32x4 sc[KS / 16];
    float tmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < KS / 16; ++t) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < DK; ++ks) {
        const int d0 = 32 * ks + 8 * gi;
        const int off = ((16 * t + c) * D + d0) * 2;
        const bf16x8 ah = d0 < D ? *(const bf16x8*)(sb + off) : zero8;
        const bf16x8 al = d0 < D ? *(const bf16x8*)(sb + kTile + off) : zero8;
        acc = mfma16bf(ah, qh[ks], acc);
        acc = mfma16bf(ah, ql[ks], acc);
        acc = mfma16bf(al, qh[ks], acc);
      }
      if (T16) {
        const int off = ((16 * t + c) * D + 32 * DK + 4 * gi) * 2;
        const bf16x4 ah = *(const bf16x4*)(sb + off), al = *(const bf16x4*)(sb + kTile + off);
        acc = mfma16bf_k16(ah, qh4, acc);
        acc = mfma16bf_k16(ah, ql4, acc);
        acc = mfma16bf_k16(al, qh4, acc);
      }
      const int kb = key0 + 16 * t + 4 * gi;  // this lane's keys kb .. kb + 3
      f32x4 b4;
      if (full) {
        b4 = *(const f32x4*)(brow + kb);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) b4[r] = brow[min(kb + r, nk - 1)];
      }
      const f32x4 m4 = *(const f32x4*)(mterm + kb);  // (1 - mask) * -inf, -inf past nk
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        sc[t][r] = (acc[r] * rscale + b4[r]) + m4[r];
        tmax = fmaxf(tmax, sc[t][r]);
      }
    }
    const float mn = fmaxf(m, col_max(tmax));
    const float alpha = __builtin_amdgcn_exp2f((m - mn) * kLog2e);
    m = mn;
    lsum *= alpha;
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] *= alpha;
#pragma unroll
    for (int s2 = 0; s2 < KS / 32; ++s2) {
      // P^T of keys key0 + 32 s2 + (slots): slot 4 t' + r <-> key 16 t' + 4 gi + r of the 32-key block
      bf16x8 ph, pl;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float pr = __builtin_amdgcn_exp2f((sc[2 * s2 + t][r] - mn) * kLog2e);
          lsum += pr;
          ph[4 * t + r] = (bf16)pr;
          pl[4 * t + r] = (bf16)(pr - (float)ph[4 * t + r]);
        }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const int d = 16 * dt + c, chunk = 4 * s2 + gi;
        const int off = d * (KS * 2) + ((chunk ^ (d & kSwz)) * 16);
        const bf16x8 vh = d < D ? *(const bf16x8*)(sb + 2 * kTile + off) : zero8;
        const bf16x8 vl = d < D ? *(const bf16x8*)(sb + 3 * kTile + off) : zero8;
        o[dt] = mfma16bf(vh, ph, o[dt]);
        o[dt] = mfma16bf(vh, pl, o[dt]);
        o[dt] = mfma16bf(vl, ph, o[dt]);
      }
    }
    wait_vm0();  // this wave's DMAs of the next stage
    __syncthreads();
  }
  // This wave holds every key of its 16 queries: O^T rows 16 dt + 4 gi + r of query qw + c.
  lsum = col_sum(lsum);
  const int i = qw + c;
  if (i < nq) {
    const float inv = 1.f / lsum;
    // op: the row as the split-bf16 operand of the next linear, [hi | hi | lo | 1 1 0 ...]
    // over 3 HD + 64 columns (the tail written by the head-0 blocks)
    bf16* orow = op ? op + ((int64_t)b * nq + i) * (3 * HD + 64) : nullptr;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int d0 = 16 * dt + 4 * gi;
      if (d0 < D) {
        const f32x4 gv = load4(g + (int64_t)i * ldq + h * D + d0);
        f32x4 r;
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = sigmoid_f(gv[e]) * (o[dt][e] * inv);
        if (orow) {
          bf16x4 hi, lo;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            hi[e] = (bf16)r[e];
            lo[e] = (bf16)(r[e] - (float)hi[e]);
          }
          *(bf16x4*)(orow + h * D + d0) = hi;
          *(bf16x4*)(orow + HD + h * D + d0) = hi;
          *(bf16x4*)(orow + 2 * HD + h * D + d0) = lo;
        } else {
          store4(out + (int64_t)i * HD + h * D + d0, r);
        }
      }
    }
    if (orow && h == 0) {  // lanes gi = 0..3 write 16 tail columns each
      bf16x8 t = {};
      if (gi == 0) t[0] = t[1] = (bf16)1.f;
      *(bf16x8*)(orow + 3 * HD + 16 * gi) = t;
      t[0] = t[1] = (bf16)0.f;
      *(bf16x8*)(orow + 3 * HD + 16 * gi + 8) = t;
    }
  }
}

size_t x3_workspace_bytes(int64_t batch, int64_t nk, int heads, int head_dim) {
  const size_t tile = (size_t)(batch * heads * head_dim * x3_nkp(nk)) * sizeof(bf16);  // K and V^T alike
  return 4 * ((tile + 255) / 256 * 256) + (size_t)(batch * x3_nkp(nk)) * sizeof(float);
}

int launch_seq_attention_x3(const char* name, const float* q, const float* k, const float* v, const float* bias,
                            const float* mask, const float* g, int64_t batch, const SeqAttnShape& sh, int heads,
                            int head_dim, float inf, float* out, bf16* op, void* ws, hipStream_t stream) {
  const int64_t hd = (int64_t)heads * head_dim, nkp = x3_nkp(sh.nk);
  const size_t tile = ((size_t)(batch * hd * nkp) * sizeof(bf16) + 255) / 256 * 256;
  bf16* kh = (bf16*)ws;
  bf16* kl = (bf16*)((char*)ws + tile);
  bf16* vth = (bf16*)((char*)ws + 2 * tile);
  bf16* vtl = (bf16*)((char*)ws + 3 * tile);
  float* mterm = (float*)((char*)ws + 4 * tile);
  const bool kvec = (uintptr_t)k % 16 == 0 && sh.ldk % 4 == 0 && sh.sk % 4 == 0;  // 16-byte K rows
  // rows of at most 128 channels: 64 keys per block (nkp is a multiple of 64)
  const int kg = hd <= 128 ? 2 : 1, span = 256 / kg;
  const dim3 sgrid((unsigned)((hd + span - 1) / span), (unsigned)(nkp / (32 * kg)), (unsigned)batch);
#define SEQ_ATTN_SPLIT(VEC, KG)                                                                                \
  seq_attn_split_kernel<VEC, KG><<<sgrid, 256, 0, stream>>>(k, v, sh.nk, sh.ldk, sh.sk, heads, head_dim, mask, \
                                                            sh.smask, inf, kh, kl, vth, vtl, mterm)
  if (kvec && kg == 2) SEQ_ATTN_SPLIT(true, 2);
  else if (kvec) SEQ_ATTN_SPLIT(true, 1);
  else if (kg == 2) SEQ_ATTN_SPLIT(false, 2);
  else SEQ_ATTN_SPLIT(false, 1);
#undef SEQ_ATTN_SPLIT
  if (int rc = check_launch(name)) return rc;
  const bool vec = sh.nk % 4 == 0 && sh.sbias % 4 == 0 && (uintptr_t)bias % 16 == 0;  // 16-byte bias rows
  const int64_t items = (batch + sh.bdiv - 1) / sh.bdiv * sh.bdiv * heads * ((sh.nq + kX3Q - 1) / kX3Q);
  const dim3 grid((unsigned)(8 * ((items + 7) / 8)));
  const float rscale = 1.f / sqrtf((float)head_dim);
#define SEQ_ATTN_X3(DIM)                                                                                       \
  seq_attention_x3_kernel<DIM><<<grid, 256, 0, stream>>>(q, kh, kl, vth, vtl, mterm, bias, g, sh, heads, batch, \
                                                         rscale, vec, out, op)
  if (head_dim == 24) SEQ_ATTN_X3(24);
  else if (head_dim == 32) SEQ_ATTN_X3(32);
  else SEQ_ATTN_X3(48);
#undef SEQ_ATTN_X3
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

int bmx_seq_attention_windowed_fwd(const float* q, const float* k, const float* v, const float* bias,
                                   const float* mask, const float* g, int64_t batch, int64_t nq, int64_t nk,
                                   int64_t ldq, int64_t ldk, int64_t windows, int64_t key_offset,
                                   int64_t bias_group, int64_t sbias_group, int64_t sbias, int64_t sbias_h,
                                   int64_t sbias_q, int64_t sbias_k, int heads, int head_dim, float inf, float* out,
                                   hipStream_t stream) {
  BMX_REQUIRE(batch >= 0 && batch <= 65535, "bmx_seq_attention_windowed_fwd: batch must be in [0, 65535]");
  BMX_REQUIRE(nq >= 1 && nq <= 4096 && nk >= 1 && nk <= 4096,
              "bmx_seq_attention_windowed_fwd: need 1 <= nq, nk <= 4096");
  BMX_REQUIRE(head_dim == 24 || head_dim == 32 || head_dim == 48,
              "bmx_seq_attention_windowed_fwd: head_dim must be 24, 32 or 48 (got %d)", head_dim);
  BMX_REQUIRE(heads >= 1 && heads <= 64, "bmx_seq_attention_windowed_fwd: heads must be in [1, 64] (got %d)",
              heads);
  BMX_REQUIRE(ldq >= (int64_t)heads * head_dim && ldk >= (int64_t)heads * head_dim,
              "bmx_seq_attention_windowed_fwd: row strides must be >= heads * head_dim");
  BMX_REQUIRE(windows >= 1 && windows * nq <= (1 << 24) && batch % windows == 0,
              "bmx_seq_attention_windowed_fwd: need windows >= 1 dividing batch, windows * nq <= 2^24");
  BMX_REQUIRE(key_offset <= 0 && key_offset + nk >= nq,
              "bmx_seq_attention_windowed_fwd: need key_offset <= 0 and key_offset + nk >= nq (every window "
              "sees its own queries)");
  BMX_REQUIRE(bias_group >= 1 && bias_group % windows == 0,
              "bmx_seq_attention_windowed_fwd: bias_group must be a positive multiple of windows");
  BMX_REQUIRE(sbias_group >= 0 && sbias >= 0 && sbias_h >= 0 && sbias_q >= 1 && sbias_k >= 0 &&
                  bias_group <= (1 << 30),
              "bmx_seq_attention_windowed_fwd: bias strides must be >= 0 (the query stride >= 1)");
  BMX_REQUIRE(inf > 0.f, "bmx_seq_attention_windowed_fwd: inf must be positive");
  if (batch == 0) return BMX_OK;
  BMX_REQUIRE(q && k && v && bias && mask && g && out, "bmx_seq_attention_windowed_fwd: null pointer");
  SeqAttnShape sh{(int)nq, (int)nk, (int)bias_group, ldq, ldk, nq * ldq, nq * ldk, sbias, nq};
  sh.bwin = (int)windows;
  sh.sbg = sbias_group;
  sh.sbh = sbias_h;
  sh.sbq = sbias_q;
  sh.sbk = sbias_k;
  sh.nw = (int)windows;
  sh.wq = (int)nq;
  sh.koff = (int)key_offset;
  return launch_seq_attention("bmx_seq_attention_windowed_fwd", q, k, v, bias, mask, g, batch, sh, heads, head_dim,
                              inf, out, stream);
}

size_t bmx_seq_attention_x3_workspace_bytes(int64_t batch, int64_t nk, int heads, int head_dim) {
  if (batch <= 0 || nk <= 0 || heads <= 0 || head_dim <= 0) return 0;
  return x3_workspace_bytes(batch, nk, heads, head_dim);
}

int bmx_seq_attention_x3_batched_fwd(const float* q, const float* k, const float* v, const float* bias,
                                     const float* mask, const float* g, int64_t batch, int64_t nq, int64_t nk,
                                     int64_t ldq, int64_t ldk, int64_t sq, int64_t sk, int64_t sbias, int64_t smask,
                                     int64_t bias_div, int heads, int head_dim, float inf, float* out,
                                     void* workspace, size_t workspace_bytes, hipStream_t stream) {
  BMX_REQUIRE(batch >= 0 && batch <= 65535, "bmx_seq_attention_x3_batched_fwd: batch must be in [0, 65535]");
  BMX_REQUIRE(nq >= 0 && nq <= (1 << 20) && nk >= 1 && nk <= (1 << 20),
              "bmx_seq_attention_x3_batched_fwd: need 0 <= nq <= 2^20 and 1 <= nk <= 2^20");
  BMX_REQUIRE(head_dim == 24 || head_dim == 32 || head_dim == 48,
              "bmx_seq_attention_x3_batched_fwd: head_dim must be 24, 32 or 48 (got %d)", head_dim);
  BMX_REQUIRE(heads >= 1 && heads <= 64, "bmx_seq_attention_x3_batched_fwd: heads must be in [1, 64] (got %d)",
              heads);
  BMX_REQUIRE(ldq >= (int64_t)heads * head_dim && ldk >= (int64_t)heads * head_dim,
              "bmx_seq_attention_x3_batched_fwd: row strides must be >= heads * head_dim");
  BMX_REQUIRE(sq >= 0 && sk >= 0 && sbias >= 0 && smask >= 0 && bias_div >= 1,
              "bmx_seq_attention_x3_batched_fwd: strides must be >= 0 and bias_div >= 1");
  BMX_REQUIRE(inf > 0.f, "bmx_seq_attention_x3_batched_fwd: inf must be positive");
  if (batch == 0 || nq == 0) return BMX_OK;
  BMX_REQUIRE(q && k && v && bias && mask && g && out && workspace,
              "bmx_seq_attention_x3_batched_fwd: null pointer");
  BMX_REQUIRE(ldq % 4 == 0 && sq % 4 == 0 && (uintptr_t)g % 16 == 0 && (uintptr_t)out % 16 == 0,
              "bmx_seq_attention_x3_batched_fwd: g and out must be 16-byte aligned, ldq and sq multiples of 4");
  const size_t need = x3_workspace_bytes(batch, nk, heads, head_dim);
  BMX_REQUIRE(workspace_bytes >= need && (uintptr_t)workspace % 256 == 0,
              "bmx_seq_attention_x3_batched_fwd: workspace must be 256-byte aligned and hold %zu bytes (got %zu)",
              need, workspace_bytes);
  const SeqAttnShape sh{(int)nq, (int)nk, (int)bias_div, ldq, ldk, sq, sk, sbias, smask};
  return launch_seq_attention_x3("bmx_seq_attention_x3_batched_fwd", q, k, v, bias, mask, g, batch, sh, heads,
                                 head_dim, inf, out, nullptr, workspace, stream);
}

int bmx_seq_attention_x3_batched_split_fwd(const float* q, const float* k, const float* v, const float* bias,
                                           const float* mask, const float* g, int64_t batch, int64_t nq, int64_t nk,
                                           int64_t ldq, int64_t ldk, int64_t sq, int64_t sk, int64_t sbias,
                                           int64_t smask, int64_t bias_div, int heads, int head_dim, float inf,
                                           void* out_op, void* workspace, size_t workspace_bytes,
                                           hipStream_t stream) {
  BMX_REQUIRE(batch >= 0 && batch <= 65535, "bmx_seq_attention_x3_batched_split_fwd: batch must be in [0, 65535]");
  BMX_REQUIRE(nq >= 0 && nq <= (1 << 20) && nk >= 1 && nk <= (1 << 20),
              "bmx_seq_attention_x3_batched_split_fwd: need 0 <= nq <= 2^20 and 1 <= nk <= 2^20");
  BMX_REQUIRE(head_dim == 24 || head_dim == 32 || head_dim == 48,
              "bmx_seq_attention_x3_batched_split_fwd: head_dim must be 24, 32 or 48 (got %d)", head_dim);
  BMX_REQUIRE(heads >= 1 && heads <= 64, "bmx_seq_attention_x3_batched_split_fwd: heads must be in [1, 64] (got %d)",
              heads);
  BMX_REQUIRE(ldq >= (int64_t)heads * head_dim && ldk >= (int64_t)heads * head_dim,
              "bmx_seq_attention_x3_batched_split_fwd: row strides must be >= heads * head_dim");
  BMX_REQUIRE(sq >= 0 && sk >= 0 && sbias >= 0 && smask >= 0 && bias_div >= 1,
              "bmx_seq_attention_x3_batched_split_fwd: strides must be >= 0 and bias_div >= 1");
  BMX_REQUIRE(inf > 0.f, "bmx_seq_attention_x3_batched_split_fwd: inf must be positive");
  if (batch == 0 || nq == 0) return BMX_OK;
  BMX_REQUIRE(q && k && v && bias && mask && g && out_op && workspace,
              "bmx_seq_attention_x3_batched_split_fwd: null pointer");
  BMX_REQUIRE(ldq % 4 == 0 && sq % 4 == 0 && (uintptr_t)g % 16 == 0 && (uintptr_t)out_op % 16 == 0,
              "bmx_seq_attention_x3_batched_split_fwd: g and out_op must be 16-byte aligned, ldq and sq multiples of 4");
  const size_t need = x3_workspace_bytes(batch, nk, heads, head_dim);
  BMX_REQUIRE(workspace_bytes >= need && (uintptr_t)workspace % 256 == 0,
              "bmx_seq_attention_x3_batched_split_fwd: workspace must be 256-byte aligned and hold %zu bytes (got %zu)",
              need, workspace_bytes);
  const SeqAttnShape sh{(int)nq, (int)nk, (int)bias_div, ldq, ldk, sq, sk, sbias, smask};
  return launch_seq_attention_x3("bmx_seq_attention_x3_batched_split_fwd", q, k, v, bias, mask, g, batch, sh, heads,
                                 head_dim, inf, nullptr, (bf16*)out_op, workspace, stream);
}

}  // extern "C"
