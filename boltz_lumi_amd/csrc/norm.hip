// LayerNorm kernels.
//
//  bmx_layernorm128   LN over exactly 128 channels, channel-last [rows,128] or
//                     channel-first [128,rows]; fp32/bf16 in, fp32/bf16 out.
//                     Replaces the reference's ``multiplication_norm``
//                     (kernels/multiplication_hip.cu:149-156).
//  bmx_layernorm      LN over D <= 1024 channels with optional weight / bias
//                     (AdaLN's a_norm without affine and s_norm without bias).
//  bmx_adaln          sigmoid(scale) * LN_noaffine(a) + shift in one pass
//  bmx_adaln_strided  the same with scale / shift rows at a stride
//                     (AdaLN.forward after the s_scale / s_bias GEMMs,
//                     reference diffusion.py:52-57 + diffusion_hip.cu:14-18).
#include "bmx_common.h"

using namespace bmx;

namespace {

// Channel-last: a half-wave per row, 4 channels per lane.
template <typename TIn, typename TOut>
__global__ __launch_bounds__(256) void ln128_rows_kernel(const TIn* __restrict__ x, const float* __restrict__ w,
                                                         const float* __restrict__ b, TOut* __restrict__ out,
                                                         int64_t rows, float eps) {
  const int hl = threadIdx.x & 31;
  const LnAffine aff = ln_affine(w, b, hl);
  const int64_t stride = (int64_t)gridDim.x * (blockDim.x >> 5);
  for (int64_t row = (int64_t)blockIdx.x * (blockDim.x >> 5) + (threadIdx.x >> 5); row < rows; row += stride) {
    f32x4 v = load4(x + row * kC + 4 * hl);
    f32x4 y = ln128_half(v, aff, eps);
    TOut* o = out + row * kC + 4 * hl;
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = (TOut)y[u];
  }
}

// Channel-first input x[c * rows + r]: a block stages 64 rows x 128 channels
// through LDS, then normalises them channel-last.
template <typename TIn, typename TOut>
__global__ __launch_bounds__(256) void ln128_cf_kernel(const TIn* __restrict__ x, const float* __restrict__ w,
                                                       const float* __restrict__ b, TOut* __restrict__ out,
                                                       int64_t rows, float eps) {
  __shared__ float tile[64][kC + 1];
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int t = threadIdx.x;
  for (int i = t; i < 64 * kC; i += 256) {
    int c = i >> 6, r = i & 63;
    tile[r][c] = (r0 + r < rows) ? load_f(x + (int64_t)c * rows + r0 + r) : 0.f;
  }
  __syncthreads();
  const int hw = t >> 5, hl = t & 31;
  const LnAffine aff = ln_affine(w, b, hl);
  for (int r = hw; r < 64; r += 8) {
    if (r0 + r >= rows) break;
    f32x4 v = {tile[r][4 * hl], tile[r][4 * hl + 1], tile[r][4 * hl + 2], tile[r][4 * hl + 3]};
    f32x4 y = ln128_half(v, aff, eps);
    TOut* o = out + (r0 + r) * kC + 4 * hl;
#pragma unroll
    for (int u = 0; u < 4; ++u) o[u] = (TOut)y[u];
  }
}

constexpr int kMaxChunks = 4;  // float4 chunks per lane -> D <= 1024

// General LayerNorm, one wave per row.
template <typename T>
__global__ __launch_bounds__(256) void ln_rows_kernel(const T* __restrict__ x, const float* __restrict__ w,
                                                      const float* __restrict__ b, T* __restrict__ out,
                                                      int64_t rows, int d, float eps) {
  const int l = lane_id();
  const int chunks = d >> 2;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  f32x4 v[kMaxChunks];
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxChunks; ++u) {
    int ch = l + 64 * u;
    v[u] = ch < chunks ? load4(x + row * d + 4 * ch) : f32x4{0.f, 0.f, 0.f, 0.f};
    s += v[u][0] + v[u][1] + v[u][2] + v[u][3];
  }
  const float mean = wave_sum_full(s) / d;
  float q = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxChunks; ++u) {
    if (l + 64 * u < chunks) {
      f32x4 dv = v[u] - mean;
      q += dv[0] * dv[0] + dv[1] * dv[1] + dv[2] * dv[2] + dv[3] * dv[3];
    }
  }
  const float inv = rsqrtf(wave_sum_full(q) / d + eps);
#pragma unroll
  for (int u = 0; u < kMaxChunks; ++u) {
    int ch = l + 64 * u;
    if (ch < chunks) {
      f32x4 y = (v[u] - mean) * inv;
      if (w) y = y * load4(w + 4 * ch);
      if (b) y = y + load4(b + 4 * ch);
#pragma unroll
      for (int e = 0; e < 4; ++e) out[row * d + 4 * ch + e] = (T)y[e];
    }
  }
}

// out = sigmoid(scale) * LN(a) + shift; multiply and add round separately as
// in the eager PyTorch expression.  LANES lanes per row: 64, or 32 for
// d <= 128 (two rows per wave, so no lane idles at the atom transformer's
// width).  a, scale and shift are all requested before the row reductions,
// with indices clamped into the row so that every load is unconditional.
// scale and shift rows sit at stride ldm (d when they are dense).
template <typename T, int LANES>
__global__ __launch_bounds__(256) void adaln_kernel(const T* __restrict__ a, const T* __restrict__ scale,
                                                    const T* __restrict__ shift, int64_t ldm, T* __restrict__ out,
                                                    int64_t rows, int d, float eps) {
#pragma clang fp contract(off)
  constexpr int kPer = LANES == 64 ? kMaxChunks : 1;  // float4 chunks per lane: d <= 4 * LANES * kPer
  const int l = threadIdx.x & (LANES - 1);
  const int chunks = d >> 2;
  const int64_t row = (int64_t)blockIdx.x * (256 / LANES) + threadIdx.x / LANES;
  if (row >= rows) return;  // whole rows (a half-wave's reductions stay inside the half-wave)
  const int64_t base = row * d;
  f32x4 v[kPer], sc[kPer], sh[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int ch = min(l + LANES * u, chunks - 1);
    v[u] = load4(a + base + 4 * ch);
    sc[u] = load4(scale + row * ldm + 4 * ch);
    sh[u] = load4(shift + row * ldm + 4 * ch);
  }
  auto reduce = [](float x) { return LANES == 64 ? wave_sum_full(x) : half_sum(x); };
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < kPer; ++u)
    if (l + LANES * u < chunks) s += v[u][0] + v[u][1] + v[u][2] + v[u][3];
  const float mean = reduce(s) / d;
  float q = 0.f;
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    if (l + LANES * u < chunks) {
      f32x4 dv = v[u] - mean;
      q += dv[0] * dv[0] + dv[1] * dv[1] + dv[2] * dv[2] + dv[3] * dv[3];
    }
  }
  const float inv = rsqrtf(reduce(q) / d + eps);
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const int ch = l + LANES * u;
    if (ch < chunks) {
      f32x4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float an = (v[u][e] - mean) * inv;
        float prod = sigmoid_f(sc[u][e]) * an;
        r[e] = prod + sh[u][e];
      }
      store4(out + base + 4 * ch, r);
    }
  }
}

template <typename TIn, typename TOut>
int launch_ln128(const void* x, int channel_first, const float* w, const float* b, float eps, void* out,
                 int64_t rows, hipStream_t st) {
  if (channel_first) {
    ln128_cf_kernel<TIn, TOut><<<dim3((unsigned)((rows + 63) / 64)), dim3(256), 0, st>>>(
        (const TIn*)x, w, b, (TOut*)out, rows, eps);
  } else {
    int64_t blocks = (rows + 7) / 8;
    if (blocks > 65536) blocks = 65536;
    ln128_rows_kernel<TIn, TOut><<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const TIn*)x, w, b, (TOut*)out,
                                                                               rows, eps);
  }
  return check_launch("bmx_layernorm128");
}

}  // namespace

extern "C" {

int bmx_layernorm128(const void* x, int x_dtype, int channel_first, const float* weight, const float* bias,
                     float eps, void* out, int out_dtype, int64_t rows, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0, "bmx_layernorm128: rows must be >= 0");
  BMX_REQUIRE(eps > 0.f, "bmx_layernorm128: eps must be positive");
  BMX_REQUIRE((x_dtype == kF32 || x_dtype == kBF16) && (out_dtype == kF32 || out_dtype == kBF16),
              "bmx_layernorm128: dtypes must be fp32 or bf16");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(x && out && weight && bias, "bmx_layernorm128: null pointer");
  BMX_REQUIRE(channel_first || ((uintptr_t)x % (x_dtype == kF32 ? 16 : 8) == 0),
              "bmx_layernorm128: x must be 16-byte (fp32) / 8-byte (bf16) aligned");
  if (x_dtype == kF32)
    return out_dtype == kF32 ? launch_ln128<float, float>(x, channel_first, weight, bias, eps, out, rows, stream)
                             : launch_ln128<float, bf16>(x, channel_first, weight, bias, eps, out, rows, stream);
  return out_dtype == kF32 ? launch_ln128<bf16, float>(x, channel_first, weight, bias, eps, out, rows, stream)
                           : launch_ln128<bf16, bf16>(x, channel_first, weight, bias, eps, out, rows, stream);
}

int bmx_layernorm(const void* x, const float* weight, const float* bias, float eps, void* out, int dtype,
                  int64_t rows, int dim, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && dim > 0 && dim % 4 == 0 && dim <= 1024,
              "bmx_layernorm: need rows >= 0 and 0 < dim <= 1024, dim %% 4 == 0 (got %d)", dim);
  BMX_REQUIRE(dtype == kF32 || dtype == kBF16, "bmx_layernorm: dtype must be fp32 or bf16");
  BMX_REQUIRE(eps > 0.f, "bmx_layernorm: eps must be positive");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(x && out, "bmx_layernorm: null pointer");
  dim3 grid((unsigned)((rows + 3) / 4));
  if (dtype == kF32)
    ln_rows_kernel<float><<<grid, 256, 0, stream>>>((const float*)x, weight, bias, (float*)out, rows, dim, eps);
  else
    ln_rows_kernel<bf16><<<grid, 256, 0, stream>>>((const bf16*)x, weight, bias, (bf16*)out, rows, dim, eps);
  return check_launch("bmx_layernorm");
}

int bmx_adaln_strided(const void* a, const void* scale, const void* shift, int64_t ld_mod, void* out, int dtype,
                      int64_t rows, int dim, float eps, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && dim > 0 && dim % 4 == 0 && dim <= 1024,
              "bmx_adaln: need 0 < dim <= 1024 and dim %% 4 == 0 (got %d)", dim);
  BMX_REQUIRE(ld_mod >= dim && ld_mod % 4 == 0, "bmx_adaln: need ld_mod >= dim and ld_mod %% 4 == 0");
  BMX_REQUIRE(dtype == kF32 || dtype == kBF16, "bmx_adaln: dtype must be fp32 or bf16");
  BMX_REQUIRE(eps > 0.f, "bmx_adaln: eps must be positive");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(a && scale && shift && out, "bmx_adaln: null pointer");
  const int align = dtype == kF32 ? 16 : 8;
  BMX_REQUIRE(((uintptr_t)a | (uintptr_t)scale | (uintptr_t)shift | (uintptr_t)out) % align == 0,
              "bmx_adaln: operands must be %d-byte aligned", align);
#define ADALN(T, LANES)                                                                             \
  adaln_kernel<T, LANES><<<dim3((unsigned)((rows + 256 / LANES - 1) / (256 / LANES))), 256, 0, stream>>>( \
      (const T*)a, (const T*)scale, (const T*)shift, ld_mod, (T*)out, rows, dim, eps)
  if (dtype == kF32) {
    if (dim <= 128) ADALN(float, 32);
    else ADALN(float, 64);
  } else {
    if (dim <= 128) ADALN(bf16, 32);
    else ADALN(bf16, 64);
  }
#undef ADALN
  return check_launch("bmx_adaln");
}

int bmx_adaln(const void* a, const void* scale, const void* shift, void* out, int dtype, int64_t rows, int dim,
              float eps, hipStream_t stream) {
  return bmx_adaln_strided(a, scale, shift, dim, out, dtype, rows, dim, eps, stream);
}

}  // extern "C"
