// Fused pair transition for gfx950: LN -> fc1 | fc2 (128 -> 512 each) ->
// bf16(bf16(silu(fc1)) * fc2) -> fc3 (512 -> 128), one kernel per 128 pairs.
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
  auto row_ptr = [&](int p) -> const TIn* { return r0 + p < rows ? x + (r0 + p) * kC : nullptr; };
  ln_rows_to_lds<kTP, TIn>(row_ptr, ln_w, ln_b, eps, xn);
  __syncthreads();

  const int c0 = 32 * w;
  f32x16 y[4] = {zero16(), zero16(), zero16(), zero16()};
  for (int hc = 0; hc < kHidden / kC; ++hc) {
    {
      bf16x8 f1[8], f2[8];
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        f1[ks] = frag(w12, kC, hc * kC + c0, ks);
        f2[ks] = frag(w12, kC, kHidden + hc * kC + c0, ks);
      }
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
        f32x16 a1 = zero16(), a2 = zero16();
#pragma unroll
        for (int ks = 0; ks < 8; ++ks) {
          bf16x8 xf = frag(xn, kLdsRow, nt * 32, ks);
          a1 = mfma32(xf, f1[ks], a1);
          a2 = mfma32(xf, f2[ks], a2);
        }
        // D[pair][hidden]: lane = hidden channel c0 + l%32.
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          hid[(nt * 32 + drow(r, l)) * kLdsRow + c0 + (l & 31)] = (bf16)(silu_f(a1[r]) * a2[r]);
        }
      }
    }
    __syncthreads();
    bf16x8 f3[8];
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) f3[ks] = frag(w3 + hc * kC, kHidden, c0, ks);
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) y[nt] = mfma32(frag(hid, kLdsRow, nt * 32, ks), f3[ks], y[nt]);
    __syncthreads();
  }
  const int ch = c0 + (l & 31);
#pragma unroll
  for (int nt = 0; nt < 4; ++nt)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      int64_t row = r0 + nt * 32 + drow(r, l);
      if (row >= rows) continue;
      float v = rbf(y[nt][r]);
      int64_t off = row * kC + ch;
      if (out_mode == 0)
        ((bf16*)out)[off] = (bf16)v;
      else if (out_mode == 1)
        ((float*)out)[off] = v;
      else if (out_mode == 2)
        ((float*)out)[off] += v;
      else
        ((float*)out)[off] = (float)x[off] + v;
    }
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
