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

__device__ __forceinline__ f32x4 mfma16f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

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

}  // extern "C"
