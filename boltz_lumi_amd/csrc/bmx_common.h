// Shared device helpers for the gfx950 (CDNA4) kernels of libbmx.
//
// Conventions used by every kernel in this library:
//  * wave64; MFMA tiles are v_mfma_f32_32x32x16_bf16 (A/B: 8 bf16 per lane,
//    C/D: 16 fp32 per lane).  Fragment layout (lane l, half h = l / 32):
//      A (M x K): row l % 32, k-slot 8*h .. 8*h+7
//      B (K x N): col l % 32, k-slot 8*h .. 8*h+7
//      D (M x N): col l % 32, register r -> row 8*(r/4) + 4*h + (r%4)
//    The hardware pairs A and B elements that sit in the same (half, slot), so
//    any consistent k-permutation between A and B gives the same product.
//  * bf16 is the compiler's __bf16; float -> bf16 rounds to nearest even
//    (v_cvt_pk_bf16_f32), matching torch's casts.
//  * All pointers are device pointers owned by the caller; kernels never
//    allocate.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace bmx {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr int kC = 128;          // pair channels (c_z)
constexpr int kLdsRow = kC + 8;  // padded LDS row (bf16 elements) for 128-wide tiles

// dtype codes shared with include/bmx.h
enum Dtype : int { kF32 = 0, kBF16 = 1 };

__device__ __forceinline__ float rbf(float x) { return (float)(bf16)x; }

// sigmoid(x) = 1 / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32; ~1 ulp each).  An IEEE division would cost ~10 VALU
// instructions, which dominated the epilogues of the fused kernels.
__device__ __forceinline__ float sigmoid_f(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }

__device__ __forceinline__ float load_f(const float* p) { return *p; }
__device__ __forceinline__ float load_f(const bf16* p) { return (float)*p; }

// 16-byte load through a global (addrspace 1) pointer.  When a source pointer
// is picked at run time the compiler can lose its address space and emit a
// flat load, which also counts against lgkmcnt: every later LDS wait then
// waits for the global load as well, serialising a prefetch with compute.
__device__ __forceinline__ bf16x8 gload8(const bf16* p) {
  return *(const __attribute__((address_space(1))) bf16x8*)p;
}

// 4 consecutive values as fp32.
__device__ __forceinline__ f32x4 load4(const float* p) { return *(const f32x4*)p; }
__device__ __forceinline__ f32x4 load4(const bf16* p) {
  bf16x4 v = *(const bf16x4*)p;
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}
__device__ __forceinline__ void store4(float* p, f32x4 v) { *(f32x4*)p = v; }
__device__ __forceinline__ void store4(bf16* p, f32x4 v) {
  *(bf16x4*)p = bf16x4{(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
}

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v_mfma_f32_16x16x4f32 (lane l, group g = l / 16): A holds A[l%16][k = g],
// B holds B[k = g][l%16], D register r holds D[4 g + r][l%16].
__device__ __forceinline__ f32x4 mfma16f32(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Max / sum over the four lanes l%16 + 16 g of a 16x16 fragment column (xor 16
// by ds_swizzle in bitmask mode, xor 32 by permlane32_swap); every lane of
// the column gets the result.
__device__ __forceinline__ float col_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F)));
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float col_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// D-fragment row of register r for this lane (see header comment).
__device__ __forceinline__ int drow(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// v from the lane selected by a DPP control word (full row / bank masks).
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

// Sum across the 32 lanes of a half-wave; every lane gets the same bits.
// Lanes within 16 exchange through DPP (VALU, no LDS round trip): quad_perm
// xor 1, quad_perm xor 2, row_half_mirror (i <-> 7-i in 8), row_mirror
// (i <-> 15-i in 16).  The last step crosses the two 16-lane rows with
// ds_swizzle in bitmask mode (xor 16).  A __shfl_xor butterfly costs one
// ds_bpermute and a full LDS wait per step.
__device__ __forceinline__ float half_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // xor 16
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
  return v;
}
// Sum over a whole wave whose 64 lanes are all active: the DPP half-wave
// sum, then the two halves' totals read into scalars (no LDS round trip).
// The result is the same in every lane.
__device__ __forceinline__ float wave_sum_full(float v) {
  v = half_sum(v);
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
  return v;
}

// Per-lane LayerNorm affine for channels 4*hl .. 4*hl+3; a null weight or
// bias acts as 1 or 0.  Load it once, outside any row loop: a conditional load
// inside an unrolled row loop gets its own basic block and a vmcnt(0) wait,
// which also waits for every prefetch in flight.
struct LnAffine {
  f32x4 w, b;
};
__device__ __forceinline__ LnAffine ln_affine(const float* w, const float* b, int hl) {
  LnAffine a;
  a.w = w ? load4(w + 4 * hl) : f32x4{1.f, 1.f, 1.f, 1.f};
  a.b = b ? load4(b + 4 * hl) : f32x4{0.f, 0.f, 0.f, 0.f};
  return a;
}

// LayerNorm over 128 channels of one row held by a half-wave: 4 values per
// lane (channels 4*hl .. 4*hl+3).  Two-pass mean/variance in fp32.
__device__ __forceinline__ f32x4 ln128_half(f32x4 v, const LnAffine& a, float eps) {
  float s = v[0] + v[1] + v[2] + v[3];
  float mean = half_sum(s) * (1.f / kC);
  f32x4 d = v - mean;
  float q = d[0] * d[0] + d[1] * d[1] + d[2] * d[2] + d[3] * d[3];
  float inv = rsqrtf(half_sum(q) * (1.f / kC) + eps);
  return d * inv * a.w + a.b;
}

// K independent half-wave sums, each step issued for all K before the next:
// the K DPP chains and the K ds_swizzle round trips overlap instead of
// waiting one after another.  Each sum is the same bits as half_sum.
template <int K>
__device__ __forceinline__ void half_sums(float (&v)[K]) {
#pragma unroll
  for (int u = 0; u < K; ++u) v[u] += dpp<0xB1>(v[u]);
#pragma unroll
  for (int u = 0; u < K; ++u) v[u] += dpp<0x4E>(v[u]);
#pragma unroll
  for (int u = 0; u < K; ++u) v[u] += dpp<0x141>(v[u]);
#pragma unroll
  for (int u = 0; u < K; ++u) v[u] += dpp<0x140>(v[u]);
  float x[K];
#pragma unroll
  for (int u = 0; u < K; ++u) x[u] = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v[u]), 0x401F));
#pragma unroll
  for (int u = 0; u < K; ++u) v[u] += x[u];
}

// ln128_half of K rows (one per element of v, all held by this half-wave),
// with the reductions of the K rows interleaved; row u is zeroed where
// keep[u] is false.  Bit for bit ln128_half per row.
template <int K>
__device__ __forceinline__ void ln128_half_rows(f32x4 (&v)[K], const bool (&keep)[K], const LnAffine& a, float eps) {
  float s[K];
#pragma unroll
  for (int u = 0; u < K; ++u) s[u] = v[u][0] + v[u][1] + v[u][2] + v[u][3];
  half_sums(s);
  float q[K];
#pragma unroll
  for (int u = 0; u < K; ++u) {
    v[u] = v[u] - s[u] * (1.f / kC);
    q[u] = v[u][0] * v[u][0] + v[u][1] * v[u][1] + v[u][2] * v[u][2] + v[u][3] * v[u][3];
  }
  half_sums(q);
#pragma unroll
  for (int u = 0; u < K; ++u) {
    const float inv = rsqrtf(q[u] * (1.f / kC) + eps);
    const f32x4 y = v[u] * inv * a.w + a.b;
#pragma unroll
    for (int c = 0; c < 4; ++c) v[u][c] = keep[u] ? y[c] : 0.f;
  }
}

template <int K>
__device__ __forceinline__ void ln128_half_rows(f32x4 (&v)[K], const LnAffine& a, float eps) {
  bool keep[K];
#pragma unroll
  for (int u = 0; u < K; ++u) keep[u] = true;
  ln128_half_rows(v, keep, a, eps);
}

// Normalise TP rows of 128 channels into an LDS tile lds[TP][kLdsRow] (bf16).
// row_ptr(p) returns the row's base pointer or nullptr for padding rows,
// which are written as zeros.  Padding rows read the valid row `safe`
// instead, so every load is unconditional: a load under a branch gets its own
// basic block and a full vmcnt wait, serialising the tile's HBM reads.
// 256 threads: each half-wave takes TP/8 rows.
template <int TP, typename TIn, typename RowPtr>
__device__ __forceinline__ void ln_rows_to_lds(RowPtr row_ptr, const TIn* safe, const float* w, const float* b,
                                               float eps, bf16* lds) {
  const int hw = threadIdx.x >> 5, hl = threadIdx.x & 31;
  const LnAffine aff = ln_affine(w, b, hl);
  constexpr int kPer = TP / 8;
  f32x4 v[kPer];
  bool ok[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const TIn* src = row_ptr(hw + 8 * u);
    ok[u] = src != nullptr;
    v[u] = load4((ok[u] ? src : safe) + 4 * hl);
  }
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    f32x4 y = ln128_half(v[u], aff, eps);
    if (!ok[u]) y = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x4 o = {(bf16)y[0], (bf16)y[1], (bf16)y[2], (bf16)y[3]};
    *(bf16x4*)(lds + (hw + 8 * u) * kLdsRow + 4 * hl) = o;
  }
}

// Output modes of the fused pair kernels (include/bmx.h).
enum OutMode : int { kOutBF16 = 0, kOutF32 = 1, kOutAccumulate = 2, kOutResidual = 3 };

constexpr int kYRow = kC + 4;  // fp32 LDS row used to re-layout results for row-wise stores

// Store 4 consecutive channels of one result row.  y is the module output
// (already rounded to bf16 precision); xres holds the same 4 input values
// when the caller has them in registers (residual modes with out aliasing x
// or out-of-place residual writes).
__device__ __forceinline__ void store_row4(void* out, int64_t off, f32x4 y, f32x4 xres, int mode, bool x_in_regs) {
  if (mode == kOutBF16) {
    bf16x4 o = {(bf16)y[0], (bf16)y[1], (bf16)y[2], (bf16)y[3]};
    *(bf16x4*)((bf16*)out + off) = o;
  } else if (mode == kOutF32) {
    *(f32x4*)((float*)out + off) = y;
  } else {
    f32x4 base = (mode == kOutAccumulate && !x_in_regs) ? *(const f32x4*)((float*)out + off) : xres;
    *(f32x4*)((float*)out + off) = base + y;
  }
}

// A or B fragment (8 bf16) for k-step ks from a row-major tile with leading
// dimension ld (elements); the fragment row is row0 + lane % 32.
__device__ __forceinline__ bf16x8 frag(const bf16* base, int ld, int row0, int ks) {
  const int l = lane_id();
  return *(const bf16x8*)(base + (row0 + (l & 31)) * ld + 16 * ks + 8 * (l >> 5));
}

// The same fragment from a matrix packed by bmx_pack_mfma_weights (cols
// columns, row0 a multiple of 32): one contiguous 1 KB run per fragment.
__device__ __forceinline__ bf16x8 pfrag(const bf16* packed, int cols, int row0, int ks) {
  return *(const bf16x8*)(packed + (((int64_t)(row0 >> 5) * (cols >> 4) + ks) * 64 + lane_id()) * 8);
}

}  // namespace bmx

// ---------------------------------------------------------------------------
// Error reporting shared by every C-ABI entry point (defined in api.hip).
// ---------------------------------------------------------------------------
namespace bmx {
int set_error(int code, const char* fmt, ...);
int check_launch(const char* what);
// Compute units of the current device (cached per device; used to size
// persistent grids).
int device_cu_count();
}  // namespace bmx

#define BMX_OK 0
#define BMX_EINVAL 1
#define BMX_EUNSUPPORTED 2
#define BMX_ELAUNCH 3

#define BMX_REQUIRE(cond, ...)                                        \
  do {                                                                \
    if (!(cond)) return ::bmx::set_error(BMX_EINVAL, __VA_ARGS__);    \
  } while (0)
