// Weight packing into MFMA A-operand order.
//
// A kernel that streams a weight matrix as v_mfma_f32_32x32x16_bf16 A
// operands reads, per instruction, 8 bf16 from each of 32 rows.  Row-major,
// that touches 32 cache lines per 1 KB; packed, every operand is one
// contiguous 1 KB run, which the vector memory path moves in 8 lines.
//
// Packed layout of a row-major bf16 W[rows][cols] (rows % 32 == 0,
// cols % 16 == 0): row tile rt = r / 32, k step ks = c / 16, lane
// l = 32 * ((c % 16) / 8) + r % 32; element (r, c) sits at
//   ((rt * (cols / 16) + ks) * 64 + l) * 8 + c % 8.
// pfrag() in bmx_common.h reads it back.
#include "bmx_common.h"

using namespace bmx;

namespace {

__global__ __launch_bounds__(256) void pack_mfma_a_kernel(const bf16* __restrict__ src, int64_t cols,
                                                          int64_t chunks, bf16* __restrict__ dst) {
  const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= chunks) return;
  const int lane = (int)(id & 63);
  const int64_t block = id >> 6, ksteps = cols / 16;
  const int64_t r = 32 * (block / ksteps) + (lane & 31);
  const int64_t c = 16 * (block % ksteps) + 8 * (lane >> 5);
  *(bf16x8*)(dst + id * 8) = *(const bf16x8*)(src + r * cols + c);
}

}  // namespace

extern "C" {

int bmx_pack_mfma_weights(const void* src, int64_t rows, int64_t cols, void* dst, hipStream_t stream) {
  BMX_REQUIRE(rows >= 0 && cols >= 0, "bmx_pack_mfma_weights: rows and cols must be >= 0");
  BMX_REQUIRE(rows % 32 == 0 && cols % 16 == 0,
              "bmx_pack_mfma_weights: rows must be a multiple of 32 and cols of 16 (got %lld x %lld)",
              (long long)rows, (long long)cols);
  if (rows == 0 || cols == 0) return BMX_OK;
  BMX_REQUIRE(src && dst, "bmx_pack_mfma_weights: null pointer");
  BMX_REQUIRE(src != dst, "bmx_pack_mfma_weights: src and dst must not overlap");
  BMX_REQUIRE((uintptr_t)src % 16 == 0 && (uintptr_t)dst % 16 == 0,
              "bmx_pack_mfma_weights: src and dst must be 16-byte aligned");
  const int64_t chunks = rows * cols / 8;
  pack_mfma_a_kernel<<<(unsigned)((chunks + 255) / 256), 256, 0, stream>>>((const bf16*)src, cols, chunks,
                                                                            (bf16*)dst);
  return check_launch("bmx_pack_mfma_weights");
}

}  // extern "C"
