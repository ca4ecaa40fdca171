// Bandwidth-bound elementwise kernels: the reference's unfused operator set,
// written for gfx950 with channel-contiguous, vectorised access.
//
//  bmx_gate            out = bf16(x * bf16(sigmoid(g)))           (multiplication_gate_hip.cu:16-25)
//  bmx_trimul_split    gate + mask -> channel-last a, b           (multiplication_gate_hip.cu:62-73)
//  bmx_trimul_pack     gate + mask -> channel-major GEMM operands (multiplication_gate_hip.cu:27-60)
//  bmx_silu_mul        out = bf16(bf16(silu(a)) * b)              (pair_hip.cu:12-40)
//  bmx_diffusion_epilogue  MODULATION / GATE / GATED_SWIGLU       (diffusion_hip.cu:14-66)
//  bmx_gated_residual  MODULATION with a strided gate operand
//  bmx_bias_softmax    softmax(round(round(s + mask) + bias))     (triangle_softmax.py:35-114)
#include "bmx_common.h"

using namespace bmx;

namespace {

__device__ __forceinline__ float gated(float x, float g) {
  // sigmoid is rounded to bf16 before the product, as PyTorch's bf16 ops do.
  return x * rbf(sigmoid_f(g));
}

__global__ __launch_bounds__(256) void gate_vec_kernel(const bf16x8* __restrict__ x, const bf16x8* __restrict__ g,
                                                       bf16x8* __restrict__ out, int64_t n8) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  bf16x8 xv = x[i], gv = g[i], o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (bf16)gated((float)xv[e], (float)gv[e]);
  out[i] = o;
}

__global__ __launch_bounds__(256) void gate_scalar_kernel(const bf16* __restrict__ x, const bf16* __restrict__ g,
                                                          bf16* __restrict__ out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (bf16)gated((float)x[i], (float)g[i]);
}

// p, g rows hold 256 projection channels at row stride `stride` (256 for
// separate projections, 512 for the joint [p_in; g_in] projection).
__global__ __launch_bounds__(256) void split_kernel(const bf16* __restrict__ p, const bf16* __restrict__ g,
                                                    const float* __restrict__ mask, bf16* __restrict__ a,
                                                    bf16* __restrict__ b, int64_t pairs, int stride) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // one thread per 8 channels
  if (i >= pairs * 16) return;
  int64_t pair = i >> 4;
  int c8 = (int)(i & 15) * 8;
  float m = mask[pair];
  const bf16* pp = p + pair * stride;
  const bf16* gg = g + pair * stride;
  bf16x8 pa = *(const bf16x8*)(pp + c8), ga = *(const bf16x8*)(gg + c8);
  bf16x8 pb = *(const bf16x8*)(pp + kC + c8), gb = *(const bf16x8*)(gg + kC + c8);
  bf16x8 oa, ob;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    oa[e] = (bf16)(rbf(gated((float)pa[e], (float)ga[e])) * m);
    ob[e] = (bf16)(rbf(gated((float)pb[e], (float)gb[e])) * m);
  }
  *(bf16x8*)(a + pair * kC + c8) = oa;
  *(bf16x8*)(b + pair * kC + c8) = ob;
}

// Channel-major operands for the per-channel product:
//   outgoing: a_cm[c][i][k] = a[i,k,c],  b_cm[c][k][j] = b[j,k,c]
//   incoming: a_cm[c][i][k] = a[k,i,c],  b_cm[c][k][j] = b[k,j,c]
// (the reference's bmm(left, right) layout, multiplication_gate_hip.cu:52-58).
// Plane row r, columns t of an operand come from pairs (r, t), or (t, r) when
// the operand is transposed (b outgoing, a incoming).  A block writes one
// 64-column segment of one plane row for all 128 channels, as trimul_proj
// writes its operand planes: each thread gates 8 channels of one source pair
// from 16-byte loads into an LDS [channel][column] tile, which leaves as
// 16-byte segment stores.
constexpr int kPackSeg = 64;

__global__ __launch_bounds__(256) void pack_kernel(const bf16* __restrict__ p, const bf16* __restrict__ g,
                                                   const float* __restrict__ mask, bf16* __restrict__ a,
                                                   bf16* __restrict__ b, int n, int stride, int outgoing) {
  __shared__ __attribute__((aligned(16))) bf16 tile[kC][kPackSeg + 8];
  const int r = blockIdx.x, t0 = blockIdx.y * kPackSeg, operand = blockIdx.z;  // operand 0: a, 1: b
  const bool transposed = (operand == 0) != (outgoing != 0);
  const int ch0 = operand * kC;  // the operand's channels within p / g rows
  for (int idx = threadIdx.x; idx < kPackSeg * (kC / 8); idx += 256) {
    const int col = idx >> 4, c8 = (idx & 15) * 8, t = t0 + col;
    bf16x8 v = {};
    if (t < n) {
      const int64_t pair = transposed ? (int64_t)t * n + r : (int64_t)r * n + t;
      const float m = mask[pair];
      const bf16x8 pv = *(const bf16x8*)(p + pair * stride + ch0 + c8);
      const bf16x8 gv = *(const bf16x8*)(g + pair * stride + ch0 + c8);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (bf16)(rbf(gated((float)pv[e], (float)gv[e])) * m);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) tile[c8 + e][col] = v[e];
  }
  __syncthreads();
  const int64_t plane = (int64_t)n * n;
  bf16* const base = operand ? b : a;
  bf16* dst = base + (int64_t)r * n + t0;
  // With n % 8 == 0 every segment start is as aligned as the operand itself:
  // 16-byte stores when that is 16-byte aligned, element stores otherwise.
  const bool vec = n % 8 == 0 && ((uintptr_t)base & 15) == 0;
  for (int idx = threadIdx.x; idx < kC * (kPackSeg / 8); idx += 256) {
    const int c = idx >> 3, col = (idx & 7) * 8;
    bf16* out = dst + c * plane + col;
    if (vec && t0 + col + 8 <= n) {
      *(bf16x8*)out = *(const bf16x8*)&tile[c][col];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (t0 + col + e < n) out[e] = tile[c][col + e];
    }
  }
}

__device__ __forceinline__ float silu_product(float a, float b) { return rbf(a / (1.f + __expf(-a))) * b; }

__global__ __launch_bounds__(256) void silu_vec_kernel(const bf16x8* __restrict__ a, const bf16x8* __restrict__ b,
                                                       bf16x8* __restrict__ out, int64_t n8) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  bf16x8 av = a[i], bv = b[i], o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (bf16)silu_product((float)av[e], (float)bv[e]);
  out[i] = o;
}

__global__ __launch_bounds__(256) void silu_scalar_kernel(const bf16* __restrict__ a, const bf16* __restrict__ b,
                                                          bf16* __restrict__ out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = (bf16)silu_product((float)a[i], (float)b[i]);
}

enum Epilogue { kModulation = 0, kGate = 1, kGatedSwiGLU = 3 };

// fp32/bf16 epilogues; products and sums round separately as in the eager
// expressions.  One thread per 4 output elements along a row of `cols`.
template <int KIND, typename T>
__global__ __launch_bounds__(256) void epilogue_kernel(const T* __restrict__ a, const T* __restrict__ b,
                                                       const T* __restrict__ c, T* __restrict__ out, int64_t rows,
                                                       int64_t cols) {
#pragma clang fp contract(off)
  const int64_t q = cols >> 2;
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * q) return;
  // Rows are contiguous (cols % 4 == 0): element 4 i of the flat arrays; only
  // the gated SwiGLU, whose a operand is twice as wide, needs the row.
  int64_t row = 0, col = 0, o = 4 * i;
  if (KIND == kGatedSwiGLU) {
    row = i / q;
    col = (i - row * q) * 4;
    o = row * cols + col;
  }
  f32x4 r;
  if (KIND == kModulation) {
    f32x4 av = load4(a + o), bv = load4(b + o), cv = load4(c + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float prod = sigmoid_f(bv[e]) * av[e];
      r[e] = prod + cv[e];
    }
  } else if (KIND == kGate) {
    f32x4 av = load4(a + o), bv = load4(b + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = sigmoid_f(av[e]) * bv[e];
  } else {
    // a holds [x_lo | x_hi] of width 2*cols; b is the a_to_b projection.
    f32x4 lo = load4(a + row * 2 * cols + col), hi = load4(a + row * 2 * cols + cols + col), bv = load4(b + o);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float act = hi[e] / (1.f + __expf(-hi[e]));
      float prod = act * lo[e];
      r[e] = prod * bv[e];
    }
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) out[o + e] = (T)r[e];
}

// out = c + sigmoid(g) * a, the MODULATION epilogue with the gate rows at
// stride ldg (a column slice of a wider projection); one wave per row.  out
// may alias c (each element is read and written by the same lane).
__global__ __launch_bounds__(256) void gated_residual_kernel(const float* __restrict__ a, const float* __restrict__ g,
                                                             int64_t ldg, const float* c, float* out, int64_t rows,
                                                             int64_t cols) {
#pragma clang fp contract(off)
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  for (int64_t col = 4 * lane; col < cols; col += 4 * kWave) {
    const int64_t o = row * cols + col;
    const f32x4 av = load4(a + o), gv = load4(g + row * ldg + col), cv = load4(c + o);
    f32x4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float prod = sigmoid_f(gv[e]) * av[e];
      r[e] = prod + cv[e];
    }
    store4(out + o, r);
  }
}

// One block (256 threads) per score row; up to 16 keys cached per thread.
template <typename T>
__global__ __launch_bounds__(256) void bias_softmax_kernel(const T* __restrict__ s, const T* __restrict__ bias,
                                                           const float* __restrict__ mask, T* __restrict__ out,
                                                           int n_i, int n_h, int n_q, int n_k,
                                                           int64_t sb, int64_t si, int64_t sh, int64_t sq, int64_t sk,
                                                           int64_t bb, int64_t bh, int64_t bq, int64_t bk,
                                                           int64_t mb, int64_t mi, int64_t mk) {
  constexpr int kItems = 16;
  __shared__ float red[4];
  int64_t row = blockIdx.x;
  int q = row % n_q;
  int h = (row / n_q) % n_h;
  int i = (row / ((int64_t)n_q * n_h)) % n_i;
  int64_t bt = row / ((int64_t)n_q * n_h * n_i);
  const T* srow = s + bt * sb + i * si + h * sh + q * sq;
  const T* brow = bias + bt * bb + h * bh + q * bq;
  const float* mrow = mask + bt * mb + i * mi;
  float v[kItems];
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < kItems; ++u) {
    int k = threadIdx.x + 256 * u;
    v[u] = -INFINITY;
    if (k < n_k) {
      float x = (float)(T)((float)srow[k * sk] + mrow[k * mk]);
      x = (float)(T)(x + (float)brow[k * bk]);
      v[u] = x;
      mx = fmaxf(mx, x);
    }
  }
  mx = wave_max(mx);
  if (lane_id() == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  __syncthreads();
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < kItems; ++u) {
    v[u] = (threadIdx.x + 256 * u < n_k) ? __expf(v[u] - mx) : 0.f;
    sum += v[u];
  }
  sum = wave_sum(sum);
  if (lane_id() == 0) red[threadIdx.x >> 6] = sum;
  __syncthreads();
  float inv = 1.f / ((red[0] + red[1]) + (red[2] + red[3]));
  T* orow = out + row * (int64_t)n_k;
#pragma unroll
  for (int u = 0; u < kItems; ++u) {
    int k = threadIdx.x + 256 * u;
    if (k < n_k) orow[k] = (T)(v[u] * inv);
  }
}

inline unsigned blocks_for(int64_t n, int per_block) { return (unsigned)((n + per_block - 1) / per_block); }

}  // namespace

extern "C" {

int bmx_gate(const void* x, const void* g, void* out, int64_t n, hipStream_t stream) {
  BMX_REQUIRE(n >= 0, "bmx_gate: n must be >= 0");
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(x && g && out, "bmx_gate: null pointer");
  bool vec = n % 8 == 0 && ((uintptr_t)x | (uintptr_t)g | (uintptr_t)out) % 16 == 0;
  if (vec)
    gate_vec_kernel<<<blocks_for(n / 8, 256), 256, 0, stream>>>((const bf16x8*)x, (const bf16x8*)g, (bf16x8*)out,
                                                                n / 8);
  else
    gate_scalar_kernel<<<blocks_for(n, 256), 256, 0, stream>>>((const bf16*)x, (const bf16*)g, (bf16*)out, n);
  return check_launch("bmx_gate");
}

int bmx_trimul_split(const void* p, const void* g, const float* mask, void* a, void* b, int64_t pairs,
                     int row_stride, hipStream_t stream) {
  BMX_REQUIRE(pairs >= 0, "bmx_trimul_split: pairs must be >= 0");
  BMX_REQUIRE(row_stride == 256 || row_stride == 512, "bmx_trimul_split: row stride must be 256 or 512");
  if (pairs == 0) return BMX_OK;
  BMX_REQUIRE(p && g && mask && a && b, "bmx_trimul_split: null pointer");
  BMX_REQUIRE(((uintptr_t)p | (uintptr_t)g | (uintptr_t)a | (uintptr_t)b) % 16 == 0,
              "bmx_trimul_split: operands must be 16-byte aligned");
  split_kernel<<<blocks_for(pairs * 16, 256), 256, 0, stream>>>((const bf16*)p, (const bf16*)g, mask, (bf16*)a,
                                                               (bf16*)b, pairs, row_stride);
  return check_launch("bmx_trimul_split");
}

int bmx_trimul_pack(const void* p, const void* g, const float* mask, void* a, void* b, int64_t n, int row_stride,
                    int outgoing, hipStream_t stream) {
  BMX_REQUIRE(n >= 0 && n <= 65535 * 16, "bmx_trimul_pack: bad n");
  BMX_REQUIRE(row_stride == 256 || row_stride == 512, "bmx_trimul_pack: row stride must be 256 or 512");
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(p && g && mask && a && b, "bmx_trimul_pack: null pointer");
  BMX_REQUIRE(((uintptr_t)p | (uintptr_t)g) % 16 == 0, "bmx_trimul_pack: p and g must be 16-byte aligned");
  dim3 grid((unsigned)n, (unsigned)((n + kPackSeg - 1) / kPackSeg), 2);
  pack_kernel<<<grid, 256, 0, stream>>>((const bf16*)p, (const bf16*)g, mask, (bf16*)a, (bf16*)b, (int)n,
                                        row_stride, outgoing);
  return check_launch("bmx_trimul_pack");
}

int bmx_silu_mul(const void* a, const void* b, void* out, int64_t n, hipStream_t stream) {
  BMX_REQUIRE(n >= 0, "bmx_silu_mul: n must be >= 0");
  if (n == 0) return BMX_OK;
  BMX_REQUIRE(a && b && out, "bmx_silu_mul: null pointer");
  bool vec = n % 8 == 0 && ((uintptr_t)a | (uintptr_t)b | (uintptr_t)out) % 16 == 0;
  if (vec)
    silu_vec_kernel<<<blocks_for(n / 8, 256), 256, 0, stream>>>((const bf16x8*)a, (const bf16x8*)b, (bf16x8*)out,
                                                                n / 8);
  else
    silu_scalar_kernel<<<blocks_for(n, 256), 256, 0, stream>>>((const bf16*)a, (const bf16*)b, (bf16*)out, n);
  return check_launch("bmx_silu_mul");
}

int bmx_diffusion_epilogue(int kind, const void* a, const void* b, const void* c, void* out, int dtype,
                           int64_t rows, int64_t cols, hipStream_t stream) {
  BMX_REQUIRE(kind == kModulation || kind == kGate || kind == kGatedSwiGLU,
              "bmx_diffusion_epilogue: kind must be 0 (modulation), 1 (gate) or 3 (gated swiglu)");
  BMX_REQUIRE(dtype == kF32 || dtype == kBF16, "bmx_diffusion_epilogue: dtype must be fp32 or bf16");
  BMX_REQUIRE(rows >= 0 && cols > 0 && cols % 4 == 0, "bmx_diffusion_epilogue: cols must be a positive multiple of 4");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(a && b && out && (kind != kModulation || c), "bmx_diffusion_epilogue: null pointer");
  const int align = dtype == kF32 ? 16 : 8;
  BMX_REQUIRE(((uintptr_t)a | (uintptr_t)b | (uintptr_t)out | (uintptr_t)(c ? c : out)) % align == 0,
              "bmx_diffusion_epilogue: operands must be %d-byte aligned", align);
  unsigned grid = blocks_for(rows * (cols / 4), 256);
#define EPI(K, T)                                                                                     \
  epilogue_kernel<K, T><<<grid, 256, 0, stream>>>((const T*)a, (const T*)b, (const T*)c, (T*)out, rows, \
                                                   cols)
  if (dtype == kF32) {
    if (kind == kModulation) EPI(kModulation, float);
    else if (kind == kGate) EPI(kGate, float);
    else EPI(kGatedSwiGLU, float);
  } else {
    if (kind == kModulation) EPI(kModulation, bf16);
    else if (kind == kGate) EPI(kGate, bf16);
    else EPI(kGatedSwiGLU, bf16);
  }
#undef EPI
  return check_launch("bmx_diffusion_epilogue");
}

int bmx_gated_residual(const float* a, const float* gate, int64_t ld_gate, const float* c, float* out, int64_t rows,
                       int64_t cols, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && cols > 0 && cols % 4 == 0 && ld_gate >= cols && ld_gate % 4 == 0,
              "bmx_gated_residual: need cols > 0, cols %% 4 == 0, ld_gate >= cols, ld_gate %% 4 == 0");
  BMX_REQUIRE(rows < (int64_t)1 << 33, "bmx_gated_residual: too many rows");
  if (rows == 0) return BMX_OK;
  BMX_REQUIRE(a && gate && c && out, "bmx_gated_residual: null pointer");
  BMX_REQUIRE(((uintptr_t)a | (uintptr_t)gate | (uintptr_t)c | (uintptr_t)out) % 16 == 0,
              "bmx_gated_residual: operands must be 16-byte aligned");
  gated_residual_kernel<<<(unsigned)((rows + 3) / 4), 256, 0, stream>>>(a, gate, ld_gate, c, out, rows, cols);
  return check_launch("bmx_gated_residual");
}

// shape = {B, I, H, Q, K}; s_strides / b_strides / m_strides are element
// strides of scores [B,I,H,Q,K], bias [B,1,H,Q,K] and mask [B,I,1,1,K].
int bmx_bias_softmax(const void* scores, const void* bias, const float* mask, void* out, int dtype,
                     const int64_t* shape, const int64_t* s_strides, const int64_t* b_strides,
                     const int64_t* m_strides, hipStream_t stream) {
  BMX_REQUIRE(dtype == kF32 || dtype == kBF16, "bmx_bias_softmax: dtype must be fp32 or bf16");
  BMX_REQUIRE(shape && s_strides && b_strides && m_strides, "bmx_bias_softmax: null shape/stride array");
  for (int d = 0; d < 5; ++d) BMX_REQUIRE(shape[d] >= 0, "bmx_bias_softmax: negative extent");
  BMX_REQUIRE(shape[4] <= 4096, "bmx_bias_softmax: at most 4096 keys (got %lld)", (long long)shape[4]);
  int64_t rows = shape[0] * shape[1] * shape[2] * shape[3];
  if (rows == 0 || shape[4] == 0) return BMX_OK;
  BMX_REQUIRE(rows < (1ll << 31), "bmx_bias_softmax: too many rows");
  BMX_REQUIRE(scores && bias && mask && out, "bmx_bias_softmax: null pointer");
#define SM(T)                                                                                               \
  bias_softmax_kernel<T><<<(unsigned)rows, 256, 0, stream>>>(                                               \
      (const T*)scores, (const T*)bias, mask, (T*)out, (int)shape[1], (int)shape[2], (int)shape[3],         \
      (int)shape[4], s_strides[0], s_strides[1], s_strides[2], s_strides[3], s_strides[4], b_strides[0],    \
      b_strides[2], b_strides[3], b_strides[4], m_strides[0], m_strides[1], m_strides[4])
  if (dtype == kF32) SM(float);
  else SM(bf16);
#undef SM
  return check_launch("bmx_bias_softmax");
}

}  // extern "C"
