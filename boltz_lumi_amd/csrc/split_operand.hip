// Split-bf16 activation operands of the near-fp32 linears, written by the
// passes that produce the activations.
//
// The diffusion blocks' fp32 linears run as one bf16 GEMM with fp32
// accumulation (hipBLASLt) of an activation row against a weight row, both
// split into bf16 high and low parts.  For k input channels an activation row
// holds kp = 3 k + 64 bf16:
//
//     [ bf16(x) | bf16(x) | bf16(x - bf16(x)) | 1 1 0 ... 0 ]
//
// and the weight row of output n holds [ Wh | Wl | Wh | bh bl 0 ... 0 ]
// (Wh = bf16(W), Wl = bf16(W - Wh), likewise for the bias b), so the product
// sums xh Wh + xh Wl + xl Wh + bh + bl: x W + b up to the dropped xl Wl term
// and the residues below the low parts, about 2^-16 relative per product.  The
// 64-column tail carries the bias into the GEMM (two ones columns) and keeps
// kp a multiple of 64, which hipBLASLt runs as fast as 3 k.
//
//  bmx_split3_bf16            x                                -> operand
//  bmx_layernorm_split3_bf16  LayerNorm without affine of x    -> operand
//  bmx_layernorm_split3_t_bf16  the same over the transposed pairs of a square frame
//  bmx_adaln_split3_bf16      sigmoid(scale) * LN(a) + shift    -> operand
//  bmx_swiglu_split3_bf16     silu(g) * x * b of one projection -> operand
//  bmx_gated_residual_adaln_split3_bf16  c + sigmoid(g) * a -> out, and the AdaLN
//                             operand of that new row
//
// None has a reference counterpart: the reference leaves these fp32 linears
// and the passes in front of them to torch (diffusion.py:52-68,
// pair_bias.py:15-36).  One wave per row, four rows per 256-thread block.
#include "bmx_common.h"

using namespace bmx;

namespace {

constexpr int kTail = 64;       // operand columns past 3 k
constexpr int kRowChunks = 4;   // float4 chunks per lane for the LayerNorm passes: rows of <= 1024 values

__device__ __forceinline__ void put_split(bf16* row, int64_t k, int64_t col, f32x4 v) {
  bf16x4 hi, lo;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    hi[e] = (bf16)v[e];
    lo[e] = (bf16)(v[e] - (float)hi[e]);
  }
  *(bf16x4*)(row + col) = hi;
  *(bf16x4*)(row + k + col) = hi;
  *(bf16x4*)(row + 2 * k + col) = lo;
}

// Columns 3 k .. 3 k + 63: lanes 0..15 write four each.
__device__ __forceinline__ void put_tail(bf16* row, int64_t k, int lane) {
  if (lane < kTail / 4) {
    const bf16 one = (bf16)(lane == 0 ? 1.f : 0.f), zero = (bf16)0.f;
    *(bf16x4*)(row + 3 * k + 4 * lane) = bf16x4{one, one, zero, zero};
  }
}

__global__ __launch_bounds__(256) void split3_kernel(const float* __restrict__ x, int64_t ldx, bf16* __restrict__ out,
                                                     int64_t rows, int64_t k) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const float* xr = x + row * ldx;
  bf16* o = out + row * (3 * k + kTail);
  for (int64_t c = 4 * lane; c < k; c += 4 * kWave) put_split(o, k, c, load4(xr + c));
  put_tail(o, k, lane);
}

// Row statistics of LayerNorm over d values held as float4 chunks
// lane + 64 u (u < kRowChunks): the two-pass mean / biased variance of the
// LayerNorm kernels in norm.hip, same summation order.
struct RowNorm {
  float mean, inv;
};
__device__ __forceinline__ RowNorm row_norm(const f32x4 (&v)[kRowChunks], int lane, int chunks, int d, float eps) {
#pragma clang fp contract(off)
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u)
    if (lane + kWave * u < chunks) s += v[u][0] + v[u][1] + v[u][2] + v[u][3];
  const float mean = wave_sum_full(s) / d;
  float q = 0.f;
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u) {
    if (lane + kWave * u < chunks) {
      const f32x4 dv = v[u] - mean;
      q += dv[0] * dv[0] + dv[1] * dv[1] + dv[2] * dv[2] + dv[3] * dv[3];
    }
  }
  return RowNorm{mean, rsqrtf(wave_sum_full(q) / d + eps)};
}

// tn > 0: the rows of x are the pairs of a tn x tn frame read transposed
// (operand row i tn + j is x row j tn + i).
__global__ __launch_bounds__(256) void layernorm_split3_kernel(const float* __restrict__ x, int64_t ldx,
                                                               bf16* __restrict__ out, int64_t rows, int d,
                                                               float eps, int64_t tn) {
#pragma clang fp contract(off)
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63, chunks = d >> 2;
  const float* xr = x + (tn ? (row % tn) * tn + row / tn : row) * ldx;
  f32x4 v[kRowChunks];
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u) v[u] = load4(xr + 4 * min(lane + kWave * u, chunks - 1));
  const RowNorm n = row_norm(v, lane, chunks, d, eps);
  bf16* o = out + row * (3 * (int64_t)d + kTail);
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u)
    if (lane + kWave * u < chunks) put_split(o, d, 4 * (lane + kWave * u), (v[u] - n.mean) * n.inv);
  put_tail(o, d, lane);
}

// sigmoid(scale) * LN(a) + shift as bmx_adaln rounds it (the product and the
// sum separately), scale and shift rows at stride ldm.
__global__ __launch_bounds__(256) void adaln_split3_kernel(const float* __restrict__ a, const float* __restrict__ scale,
                                                           const float* __restrict__ shift, int64_t ldm,
                                                           bf16* __restrict__ out, int64_t rows, int d, float eps) {
#pragma clang fp contract(off)
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63, chunks = d >> 2;
  f32x4 v[kRowChunks], sc[kRowChunks], sh[kRowChunks];
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u) {
    const int c = 4 * min(lane + kWave * u, chunks - 1);
    v[u] = load4(a + row * d + c);
    sc[u] = load4(scale + row * ldm + c);
    sh[u] = load4(shift + row * ldm + c);
  }
  const RowNorm n = row_norm(v, lane, chunks, d, eps);
  bf16* o = out + row * (3 * (int64_t)d + kTail);
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u) {
    if (lane + kWave * u < chunks) {
      f32x4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float an = (v[u][e] - n.mean) * n.inv;
        const float prod = sigmoid_f(sc[u][e]) * an;
        r[e] = prod + sh[u][e];
      }
      put_split(o, d, 4 * (lane + kWave * u), r);
    }
  }
  put_tail(o, d, lane);
}

// The residual update of a diffusion layer and the next AdaLN in one pass:
// r = c + sigmoid(g) * a (the MODULATION epilogue; g and the modulation rows at
// strides ldg / ldm) is written to out (which may alias c), then the operand
// row of sigmoid(scale) * LN(r) + shift, rounded as bmx_adaln_split3_bf16.
__global__ __launch_bounds__(256) void gated_residual_adaln_split3_kernel(
    const float* __restrict__ a, const float* __restrict__ g, int64_t ldg, const float* c, float* out,
    const float* __restrict__ scale, const float* __restrict__ shift, int64_t ldm, bf16* __restrict__ op,
    int64_t rows, int d, float eps) {
#pragma clang fp contract(off)
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63, chunks = d >> 2;
  f32x4 v[kRowChunks], sc[kRowChunks], sh[kRowChunks];
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u) {
    const int col = 4 * min(lane + kWave * u, chunks - 1);
    const f32x4 av = load4(a + row * d + col), gv = load4(g + row * ldg + col), cv = load4(c + row * d + col);
    sc[u] = load4(scale + row * ldm + col);
    sh[u] = load4(shift + row * ldm + col);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float prod = sigmoid_f(gv[e]) * av[e];
      v[u][e] = prod + cv[e];
    }
  }
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u)
    if (lane + kWave * u < chunks) store4(out + row * d + 4 * (lane + kWave * u), v[u]);
  const RowNorm n = row_norm(v, lane, chunks, d, eps);
  bf16* o = op + row * (3 * (int64_t)d + kTail);
#pragma unroll
  for (int u = 0; u < kRowChunks; ++u) {
    if (lane + kWave * u < chunks) {
      f32x4 r;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float an = (v[u][e] - n.mean) * n.inv;
        const float prod = sigmoid_f(sc[u][e]) * an;
        r[e] = prod + sh[u][e];
      }
      put_split(o, d, 4 * (lane + kWave * u), r);
    }
  }
  put_tail(o, d, lane);
}

// Row r of u holds [x | g | b] (3 cols values at stride ldu): the swish gate's
// two halves and the a_to_b projection of the conditioned transition.  The
// operand row is silu(g) * x * b, rounded as the GATED_SWIGLU epilogue.
__global__ __launch_bounds__(256) void swiglu_split3_kernel(const float* __restrict__ u, int64_t ldu,
                                                            bf16* __restrict__ out, int64_t rows, int64_t cols) {
#pragma clang fp contract(off)
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const float* ur = u + row * ldu;
  bf16* o = out + row * (3 * cols + kTail);
  for (int64_t c = 4 * lane; c < cols; c += 4 * kWave) {
    const f32x4 x = load4(ur + c), g = load4(ur + cols + c), b = load4(ur + 2 * cols + c);
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float act = g[e] / (1.f + __expf(-g[e]));
      const float prod = act * x[e];
      r[e] = prod * b[e];
    }
    put_split(o, cols, c, r);
  }
  put_tail(o, cols, lane);
}

inline unsigned row_blocks(int64_t rows) { return (unsigned)((rows + 3) / 4); }

}  // namespace

extern "C" {

int bmx_split3_bf16(const float* x, int64_t rows, int64_t k, int64_t ldx, void* out, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && k > 0 && k % 4 == 0 && ldx >= k && ldx % 4 == 0,
              "bmx_split3_bf16: need k > 0, k %% 4 == 0, ldx >= k, ldx %% 4 == 0");
  BMX_REQUIRE(rows < (int64_t)1 << 33, "bmx_split3_bf16: too many rows");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(x && out, "bmx_split3_bf16: null pointer");
  BMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)out % 8 == 0,
              "bmx_split3_bf16: x must be 16-byte and out 8-byte aligned");
  split3_kernel<<<row_blocks(rows), 256, 0, stream>>>(x, ldx, (bf16*)out, rows, k);
  return check_launch("bmx_split3_bf16");
}

int bmx_layernorm_split3_bf16(const float* x, int64_t rows, int dim, int64_t ldx, float eps, void* out,
                              hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && dim > 0 && dim % 4 == 0 && dim <= 4 * kWave * kRowChunks && ldx >= dim && ldx % 4 == 0,
              "bmx_layernorm_split3_bf16: need 0 < dim <= 1024, dim %% 4 == 0, ldx >= dim, ldx %% 4 == 0");
  BMX_REQUIRE(eps > 0.f, "bmx_layernorm_split3_bf16: eps must be positive");
  BMX_REQUIRE(rows < (int64_t)1 << 33, "bmx_layernorm_split3_bf16: too many rows");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(x && out, "bmx_layernorm_split3_bf16: null pointer");
  BMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)out % 8 == 0,
              "bmx_layernorm_split3_bf16: x must be 16-byte and out 8-byte aligned");
  layernorm_split3_kernel<<<row_blocks(rows), 256, 0, stream>>>(x, ldx, (bf16*)out, rows, dim, eps, 0);
  return check_launch("bmx_layernorm_split3_bf16");
}

int bmx_layernorm_split3_t_bf16(const float* x, int64_t n, int dim, int64_t ldx, float eps, void* out,
                                hipStream_t stream) {
  BMX_REQUIRE(n >= 0 && dim > 0 && dim % 4 == 0 && dim <= 4 * kWave * kRowChunks && ldx >= dim && ldx % 4 == 0,
              "bmx_layernorm_split3_t_bf16: need 0 < dim <= 1024, dim %% 4 == 0, ldx >= dim, ldx %% 4 == 0");
  BMX_REQUIRE(eps > 0.f, "bmx_layernorm_split3_t_bf16: eps must be positive");
  BMX_REQUIRE(n < (int64_t)1 << 16, "bmx_layernorm_split3_t_bf16: n must be < 65536");
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(x && out, "bmx_layernorm_split3_t_bf16: null pointer");
  BMX_REQUIRE((uintptr_t)x % 16 == 0 && (uintptr_t)out % 8 == 0,
              "bmx_layernorm_split3_t_bf16: x must be 16-byte and out 8-byte aligned");
  layernorm_split3_kernel<<<row_blocks(n * n), 256, 0, stream>>>(x, ldx, (bf16*)out, n * n, dim, eps, n);
  return check_launch("bmx_layernorm_split3_t_bf16");
}

int bmx_adaln_split3_bf16(const float* a, const float* scale, const float* shift, int64_t ld_mod, int64_t rows,
                          int dim, float eps, void* out, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && dim > 0 && dim % 4 == 0 && dim <= 4 * kWave * kRowChunks && ld_mod >= dim &&
                  ld_mod % 4 == 0,
              "bmx_adaln_split3_bf16: need 0 < dim <= 1024, dim %% 4 == 0, ld_mod >= dim, ld_mod %% 4 == 0");
  BMX_REQUIRE(eps > 0.f, "bmx_adaln_split3_bf16: eps must be positive");
  BMX_REQUIRE(rows < (int64_t)1 << 33, "bmx_adaln_split3_bf16: too many rows");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(a && scale && shift && out, "bmx_adaln_split3_bf16: null pointer");
  BMX_REQUIRE(((uintptr_t)a | (uintptr_t)scale | (uintptr_t)shift) % 16 == 0 && (uintptr_t)out % 8 == 0,
              "bmx_adaln_split3_bf16: a, scale, shift must be 16-byte and out 8-byte aligned");
  adaln_split3_kernel<<<row_blocks(rows), 256, 0, stream>>>(a, scale, shift, ld_mod, (bf16*)out, rows, dim, eps);
  return check_launch("bmx_adaln_split3_bf16");
}

int bmx_gated_residual_adaln_split3_bf16(const float* a, const float* gate, int64_t ld_gate, const float* c,
                                         float* out, const float* scale, const float* shift, int64_t ld_mod,
                                         int64_t rows, int dim, float eps, void* op, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && dim > 0 && dim % 4 == 0 && dim <= 4 * kWave * kRowChunks && ld_gate >= dim &&
                  ld_gate % 4 == 0 && ld_mod >= dim && ld_mod % 4 == 0,
              "bmx_gated_residual_adaln_split3_bf16: need 0 < dim <= 1024, dim %% 4 == 0, ld_gate and ld_mod >= dim "
              "and multiples of 4");
  BMX_REQUIRE(eps > 0.f, "bmx_gated_residual_adaln_split3_bf16: eps must be positive");
  BMX_REQUIRE(rows < (int64_t)1 << 33, "bmx_gated_residual_adaln_split3_bf16: too many rows");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(a && gate && c && out && scale && shift && op, "bmx_gated_residual_adaln_split3_bf16: null pointer");
  BMX_REQUIRE(((uintptr_t)a | (uintptr_t)gate | (uintptr_t)c | (uintptr_t)out | (uintptr_t)scale | (uintptr_t)shift) %
                      16 == 0 &&
                  (uintptr_t)op % 8 == 0,
              "bmx_gated_residual_adaln_split3_bf16: fp32 operands must be 16-byte and op 8-byte aligned");
  gated_residual_adaln_split3_kernel<<<row_blocks(rows), 256, 0, stream>>>(a, gate, ld_gate, c, out, scale, shift,
                                                                           ld_mod, (bf16*)op, rows, dim, eps);
  return check_launch("bmx_gated_residual_adaln_split3_bf16");
}

int bmx_swiglu_split3_bf16(const float* u, int64_t ldu, int64_t rows, int64_t cols, void* out, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && cols > 0 && cols % 4 == 0 && ldu >= 3 * cols && ldu % 4 == 0,
              "bmx_swiglu_split3_bf16: need cols > 0, cols %% 4 == 0, ldu >= 3 cols, ldu %% 4 == 0");
  BMX_REQUIRE(rows < (int64_t)1 << 33, "bmx_swiglu_split3_bf16: too many rows");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(u && out, "bmx_swiglu_split3_bf16: null pointer");
  BMX_REQUIRE((uintptr_t)u % 16 == 0 && (uintptr_t)out % 8 == 0,
              "bmx_swiglu_split3_bf16: u must be 16-byte and out 8-byte aligned");
  swiglu_split3_kernel<<<row_blocks(rows), 256, 0, stream>>>(u, ldu, (bf16*)out, rows, cols);
  return check_launch("bmx_swiglu_split3_bf16");
}

}  // extern "C"
