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

template <typename TIn>
__global__ __launch_bounds__(256) void pair_transition_kernel(const TIn* x, const float* __restrict__ ln_w,
                                                              const float* __restrict__ ln_b, float eps,
                                                              const bf16* __restrict__ w12,
                                                              const bf16* __restrict__ w3, void* out, int out_mode,
                                                              int64_t rows) {
  __shared__ __attribute__((aligned(16))) bf16 xn[kTP * kLdsRow];
  __shared__ __attribute__((aligned(16))) bf16 hid[kTP * kLdsRow];
  const int64_t r0 = (int64_t)blockIdx.x * kTP;
  const int t = threadIdx.x, l = lane_id(), w = t >> 6;
  const int c0 = 32 * w;  // this wave's 32 hidden channels of each chunk / 32 output channels
  // fc1 / fc2 rows of one 128-wide hidden chunk (A operands).  Chunk 0 is
  // requested before the LayerNorm and chunk c+1 before the fc3 phase of
  // chunk c, so the L2 latency of the weight stream is never waited on.
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
    if (hc + 1 < kHidden / kC) load_w12(hc + 1);
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
  if (r0 + kTP <= rows)
    store_tile<true>(y, x, out, base, out_mode, r0, rows);
  else
    store_tile<false>(y, x, out, base, out_mode, r0, rows);
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
  const unsigned grid = (unsigned)((rows + kTP - 1) / kTP);
  if (x_dtype == kF32)
    pair_transition_kernel<float><<<grid, 256, 0, stream>>>((const float*)x, ln_w, ln_b, eps, (const bf16*)w12,
                                                            (const bf16*)w3, out, out_mode, rows);
  else
    pair_transition_kernel<bf16><<<grid, 256, 0, stream>>>((const bf16*)x, ln_w, ln_b, eps, (const bf16*)w12,
                                                           (const bf16*)w3, out, out_mode, rows);
  return check_launch("bmx_pair_transition_fwd");
}

}  // extern "C"
