// Fused pair transition for gfx950: LN -> fc1 | fc2 (128 -> 512 each) ->
// bf16(silu(fc1) * fc2) -> fc3 (512 -> 128), one block per 128 pairs.  The
// weights arrive packed in MFMA A-operand order (bmx_pack_mfma_weights):
// every tile streams all 384 KB of them, and packed operands are contiguous
// 1 KB loads.
//
// Replaces the reference's transition_forward (pair_transition.py:8-28:
// module.norm, fc1, fc2, the HIP silu_mul of kernels/pair_hip.cu:42-64, fc3).
// The 512-wide hidden activation never leaves the CU: it is produced in four
// 128-wide chunks into LDS and immediately contracted by fc3, whose fp32
// accumulators stay in registers across the chunks.
#include "bmx_common.h"

using namespace bmx;

namespace {

constexpr int kTP = 128, kHidden = 512;

// Write the 128 x 128 result tile held as y[nt] (D[pair][out], lane -> output
// channel, register r -> pair nt*32 + drow(r, lane)).  Residual modes load
// all 64 base values before the first store: interleaving each load with the
// previous store would serialise them on the possible out / x alias.  FULL
// tiles skip the row checks; the last tile clamps loads and masks stores.
template <bool FULL, typename TIn>
__device__ __forceinline__ void store_tile(f32x16 (&y)[4], const TIn* x, void* out, const float* base, int out_mode,
                                           int64_t r0, int64_t rows) {
  const int l = lane_id();
  const int64_t lane_off = base - (const float*)out;  // row (r0 + 4 h) * kC + channel
  auto offset = [&](int nt, int r) -> int64_t {
    const int d = (nt * 32 + 8 * (r >> 2) + (r & 3)) * kC;
    if (FULL) return lane_off + d;
    const int64_t row = min(r0 + nt * 32 + drow(r, l), rows - 1);
    return row * kC + (lane_off % kC);
  };
  if (out_mode == kOutAccumulate) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) y[nt][r] += ((const float*)out)[offset(nt, r)];
  } else if (out_mode == kOutResidual) {
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) y[nt][r] += (float)x[offset(nt, r)];
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (!FULL && r0 + nt * 32 + drow(r, l) >= rows) continue;
      if (out_mode == kOutBF16)
        ((bf16*)out)[offset(nt, r)] = (bf16)y[nt][r];
      else
        ((float*)out)[offset(nt, r)] = y[nt][r];
    }
}

// Optional epilogue: the Pairformer sequence stack's pair bias of the
// updated rows, pb_out[h][row] = sum_c LN(z_new[row])[c] * w[h][c] for 16
// heads in fp32 (upstream AttentionPairBias.proj_z, which reads z right after
// this residual add; math as pair_bias.py:21-36), so z is not read again.
// With LN(z)[c] = (z[c] - mu) * rstd * ln_w[c] + ln_b[c],
//   bias[h] = rstd * sum_c (z[c] - mu) * W'[h][c] + b[h],
//   W'[h][c] = ln_w[c] * w[h][c],  b[h] = sum_c ln_b[c] * w[h][c].
// W' and b are folded once per weight version (bmx_pair_bias_fold) into
//   hi[q][lane][8], lo[q][lane][8]: bf16 high / low parts of W'[l%16][32q + 8(l/16) + e]
//   b[16] fp32,
// the order in which the epilogue's MFMA consumes them (one 16-byte load per
// lane and k step).
struct PairBiasArgs {
  const bf16* fold;  // hi (4 KB), lo (4 KB), b (64 B)
  float eps;
  float* out;  // [16][rows]
};
constexpr int kFoldHalf = 4 * kWave * 8;  // bf16 elements in hi (and in lo)
constexpr size_t kFoldBytes = 2 * kFoldHalf * sizeof(bf16) + 16 * sizeof(float);

constexpr int kZRow = kC + 8;  // fp32 LDS row of the updated tile: 4 rows apart = 32 banks apart

// Row p of the tile's 128 updated fp32 rows: rows 0..63 over xn, 64..127 over hid.
__device__ __forceinline__ float* zrow(bf16* xn, bf16* hid, int p) {
  return (float*)(p < 64 ? xn : hid) + (p & 63) * kZRow;
}

// The rows are never normalised in place.  Wave w takes rows 32w .. 32w+31
// as two 16-row tiles; lane (row l%16, group g) reads channels 32q + 8g .. +7
// of its row (two 16-byte LDS loads per k step q); mu and the centred
// variance come from in-lane sums and the xor-16 / xor-32 exchanges.  The
// 128 -> 16 product runs on bf16 MFMA (16x16x32) with both operands split
// into bf16 high and low parts, x W' = xh Wh + xh Wl + xl Wh, which keeps
// the fp32 result to ~2^-17 relative per term at 3 MFMA per k step, instead
// of 8 fp32 MFMA (16x16x4f32) at twice the cycles each.
__device__ __forceinline__ f32x4 mfma16bf(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void split_bf16(const f32x4& a, const f32x4& b, bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = (bf16)a[e];
    hi[4 + e] = (bf16)b[e];
    lo[e] = (bf16)(a[e] - (float)hi[e]);
    lo[4 + e] = (bf16)(b[e] - (float)hi[4 + e]);
  }
}

// Folded weights of this lane: loaded before the tile's output stores, since
// a wait for a later load would also wait for those stores (vmcnt counts both).
struct PairBiasFrags {
  bf16x8 wh[4], wl[4];
  f32x4 bo;  // b[4g + r] for the D rows this lane holds
};
__device__ __forceinline__ PairBiasFrags load_pair_bias_frags(const bf16* fold) {
  const int l = lane_id();
  PairBiasFrags f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    f.wh[q] = gload8(fold + (q * kWave + l) * 8);
    f.wl[q] = gload8(fold + kFoldHalf + (q * kWave + l) * 8);
  }
  f.bo = load4((const float*)(fold + 2 * kFoldHalf) + 4 * (l >> 4));
  return f;
}

__device__ __forceinline__ void pair_bias_epilogue(bf16* xn, bf16* hid, const PairBiasFrags& f,
                                                   const PairBiasArgs& pb, int64_t r0, int64_t rows) {
  const int l = lane_id(), w = threadIdx.x >> 6, g = l >> 4, hc = l & 15;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float* row = zrow(xn, hid, 32 * w + 16 * j + hc) + 8 * g;
    f32x4 xv[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) xv[2 * q] = *(const f32x4*)(row + 32 * q), xv[2 * q + 1] = *(const f32x4*)(row + 32 * q + 4);
    float sum = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) sum += (xv[u][0] + xv[u][1]) + (xv[u][2] + xv[u][3]);
    const float mu = col_sum(sum) * (1.f / kC);
    float sq = 0.f;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      xv[u] -= mu;
#pragma unroll
      for (int e = 0; e < 4; ++e) sq = fmaf(xv[u][e], xv[u][e], sq);
    }
    const float rstd = rsqrtf(col_sum(sq) * (1.f / kC) + pb.eps);
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16x8 xh, xl;
      split_bf16(xv[2 * q], xv[2 * q + 1], xh, xl);
      acc0 = mfma16bf(f.wh[q], xh, acc0);
      acc1 = mfma16bf(f.wl[q], xh, acc1);
      acc1 = mfma16bf(f.wh[q], xl, acc1);
    }
    const int64_t grow = r0 + 32 * w + 16 * j + hc;
    if (grow < rows) {
#pragma unroll
      for (int r = 0; r < 4; ++r) pb.out[(int64_t)(4 * g + r) * rows + grow] = fmaf(rstd, acc0[r] + acc1[r], f.bo[r]);
    }
  }
}

// Fold LN affine and projection into hi / lo / b (layout above); 256 threads.
__global__ __launch_bounds__(256) void pair_bias_fold_kernel(const float* __restrict__ ln_w,
                                                             const float* __restrict__ ln_b,
                                                             const float* __restrict__ w, bf16* __restrict__ fold) {
  const int t = threadIdx.x, q = t >> 6, l = t & 63, h = l & 15, c0 = 32 * q + 8 * (l >> 4);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float v = ln_w[c0 + e] * w[h * kC + c0 + e];
    const bf16 hi = (bf16)v;
    fold[t * 8 + e] = hi;
    fold[kFoldHalf + t * 8 + e] = (bf16)(v - (float)hi);
  }
  if (t < 16) {
    float b = 0.f;
    for (int c = 0; c < kC; ++c) b = fmaf(ln_b[c], w[t * kC + c], b);
    ((float*)(fold + 2 * kFoldHalf))[t] = b;
  }
}

template <typename TIn, bool BIAS>
__global__ __launch_bounds__(256, 2) void pair_transition_kernel(const TIn* x, const float* __restrict__ ln_w,
                                                              const float* __restrict__ ln_b, float eps,
                                                              const bf16* __restrict__ w12,
                                                              const bf16* __restrict__ w3, void* out, int out_mode,
                                                              int64_t rows, PairBiasArgs pb) {
  __shared__ __attribute__((aligned(16))) bf16 xn[kTP * kLdsRow];
  __shared__ __attribute__((aligned(16))) bf16 hid[kTP * kLdsRow];
  static_assert(2 * kLdsRow * sizeof(bf16) == kZRow * sizeof(float), "64 fp32 rows must fit xn, 64 hid");
  const int64_t r0 = (int64_t)blockIdx.x * kTP;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6;
  const int c0 = 32 * w;  // this wave's 32 hidden channels of each chunk / 32 output channels
  // fc1 / fc2 rows of one 128-wide hidden chunk (A operands).  Chunk 0 is
  // requested before the LayerNorm and chunk c+1 right after the last fc1 |
  // fc2 MFMAs of chunk c, so the last SiLU products and the fc3 phase of
  // chunk c cover the L2 latency of the weight stream.
  bf16x8 f1[8], f2[8];
  auto load_w12 = [&](int hc) {
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      f1[ks] = pfrag(w12, kC, hc * kC + c0, ks);
      f2[ks] = pfrag(w12, kC, kHidden + hc * kC + c0, ks);
    }
  };
  load_w12(0);
  auto row_ptr = [&](int p) -> const TIn* { return r0 + p < rows ? x + (r0 + p) * kC : nullptr; };
  ln_rows_to_lds<kTP, TIn>(row_ptr, x + r0 * kC, ln_w, ln_b, eps, xn);
  __syncthreads();

  f32x16 y[4] = {zero16(), zero16(), zero16(), zero16()};
  for (int hc = 0; hc < kHidden / kC; ++hc) {
    bf16x8 f3[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) f3[ks] = pfrag(w3, kHidden, c0, 8 * hc + ks);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      f32x16 a1 = zero16(), a2 = zero16();
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const bf16x8 xf = frag(xn, kLdsRow, nt * 32, ks);
        a1 = mfma32(f1[ks], xf, a1);
        a2 = mfma32(f2[ks], xf, a2);
      }
      if (nt == 3 && hc + 1 < kHidden / kC) load_w12(hc + 1);
      // D[hidden][pair]: lane -> pair nt*32 + l%32, registers 4q..4q+3 ->
      // hidden channels c0 + 8q + 4(l/32) + 0..3, stored as one 8-byte write.
      bf16* dst = hid + (nt * 32 + (l & 31)) * kLdsRow + c0 + 4 * (l >> 5);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const bf16x4 v = {(bf16)(silu_f(a1[4 * q]) * a2[4 * q]), (bf16)(silu_f(a1[4 * q + 1]) * a2[4 * q + 1]),
                          (bf16)(silu_f(a1[4 * q + 2]) * a2[4 * q + 2]),
                          (bf16)(silu_f(a1[4 * q + 3]) * a2[4 * q + 3])};
        *(bf16x4*)(dst + 8 * q) = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) y[nt] = mfma32(frag(hid, kLdsRow, nt * 32, ks), f3[ks], y[nt]);
    __syncthreads();
  }
  // D[pair][out]: lane -> output channel c0 + l%32, register r -> pair
  // nt*32 + drow(r, l).
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int r = 0; r < 16; ++r) y[nt][r] = rbf(y[nt][r]);
  const float* base = (const float*)out + (r0 + 4 * (l >> 5)) * kC + c0 + (l & 31);
  PairBiasFrags pbf;
  if constexpr (BIAS) pbf = load_pair_bias_frags(pb.fold);
  if (r0 + kTP <= rows)
    store_tile<true>(y, x, out, base, out_mode, r0, rows);
  else
    store_tile<false>(y, x, out, base, out_mode, r0, rows);
  if constexpr (BIAS) {
    // y now holds the stored fp32 rows (residual included); the loop's last
    // barrier has released xn / hid.
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) zrow(xn, hid, nt * 32 + drow(r, l))[c0 + (l & 31)] = y[nt][r];
    __syncthreads();
    pair_bias_epilogue(xn, hid, pbf, pb, r0, rows);
  }
}

template <bool BIAS>
int launch_transition(const char* name, const void* x, int x_dtype, int64_t rows, const float* ln_w,
                      const float* ln_b, float eps, const void* w12, const void* w3, void* out, int out_mode,
                      const PairBiasArgs& pb, hipStream_t stream) {
  const unsigned grid = (unsigned)((rows + kTP - 1) / kTP);
  if (x_dtype == kF32)
    pair_transition_kernel<float, BIAS><<<grid, 256, 0, stream>>>((const float*)x, ln_w, ln_b, eps,
                                                                  (const bf16*)w12, (const bf16*)w3, out, out_mode,
                                                                  rows, pb);
  else
    pair_transition_kernel<bf16, BIAS><<<grid, 256, 0, stream>>>((const bf16*)x, ln_w, ln_b, eps, (const bf16*)w12,
                                                                 (const bf16*)w3, out, out_mode, rows, pb);
  return check_launch(name);
}

}  // namespace

extern "C" {

int bmx_pair_transition_fwd(const void* x, int x_dtype, int64_t rows, const float* ln_w, const float* ln_b, float eps,
                            const void* w12, const void* w3, void* out, int out_mode, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0, "bmx_pair_transition_fwd: rows must be >= 0");
  BMX_REQUIRE(x_dtype == kF32 || x_dtype == kBF16, "bmx_pair_transition_fwd: x dtype must be fp32 or bf16");
  BMX_REQUIRE(out_mode >= 0 && out_mode <= 3,
              "bmx_pair_transition_fwd: out_mode must be 0 (bf16), 1 (fp32), 2 (fp32 +=) or 3 (fp32 x + y)");
  BMX_REQUIRE(out_mode != 2 || x_dtype == kF32, "bmx_pair_transition_fwd: residual mode needs fp32 x");
  BMX_REQUIRE(eps > 0.f, "bmx_pair_transition_fwd: eps must be positive");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(x && ln_w && ln_b && w12 && w3 && out, "bmx_pair_transition_fwd: null pointer");
  BMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)w12 % 16 == 0 && (uintptr_t)w3 % 16 == 0,
              "bmx_pair_transition_fwd: x and weights must be 16-byte aligned");
  return launch_transition<false>("bmx_pair_transition_fwd", x, x_dtype, rows, ln_w, ln_b, eps, w12, w3, out,
                                  out_mode, PairBiasArgs{}, stream);
}

size_t bmx_pair_bias_fold_bytes(void) { return kFoldBytes; }

int bmx_pair_bias_fold(const float* ln_w, const float* ln_b, const float* w, int heads, void* folded,
                       hipStream_t stream) {
  BMX_REQUIRE(heads == 16, "bmx_pair_bias_fold: built for 16 heads (got %d)", heads);
  BMX_REQUIRE(ln_w && ln_b && w && folded, "bmx_pair_bias_fold: null pointer");
  BMX_REQUIRE((uintptr_t)folded % 16 == 0, "bmx_pair_bias_fold: folded must be 16-byte aligned");
  pair_bias_fold_kernel<<<1, 256, 0, stream>>>(ln_w, ln_b, w, (bf16*)folded);
  return check_launch("bmx_pair_bias_fold");
}

int bmx_pair_transition_bias_fwd(const void* x, int x_dtype, int64_t rows, const float* ln_w, const float* ln_b,
                                 float eps, const void* w12, const void* w3, void* out, int out_mode,
                                 const void* pb_folded, float pb_eps, float* pb_out, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0, "bmx_pair_transition_bias_fwd: rows must be >= 0");
  BMX_REQUIRE(x_dtype == kF32 || x_dtype == kBF16, "bmx_pair_transition_bias_fwd: x dtype must be fp32 or bf16");
  BMX_REQUIRE(out_mode >= 1 && out_mode <= 3,
              "bmx_pair_transition_bias_fwd: out_mode must be 1 (fp32), 2 (fp32 +=) or 3 (fp32 x + y)");
  BMX_REQUIRE(out_mode != 2 || x_dtype == kF32, "bmx_pair_transition_bias_fwd: residual mode needs fp32 x");
  BMX_REQUIRE(eps > 0.f && pb_eps > 0.f, "bmx_pair_transition_bias_fwd: eps must be positive");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(x && ln_w && ln_b && w12 && w3 && out && pb_folded && pb_out,
              "bmx_pair_transition_bias_fwd: null pointer");
  BMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)w12 % 16 == 0 && (uintptr_t)w3 % 16 == 0 &&
                  (uintptr_t)pb_folded % 16 == 0,
              "bmx_pair_transition_bias_fwd: x and weights must be 16-byte aligned");
  return launch_transition<true>("bmx_pair_transition_bias_fwd", x, x_dtype, rows, ln_w, ln_b, eps, w12, w3, out,
                                 out_mode, PairBiasArgs{(const bf16*)pb_folded, pb_eps, pb_out}, stream);
}

}  // extern "C"
