// Weight preparation on the device: the compiler's conversions of a layer's
// weights into WBUF DDR words (tools/compiler/tensors.cpp:66-90 PackWbuf), for
// a runtime that loads checkpoints straight into GPU memory.
//   W8:    PadRows, EncodeMxint8, SplitW8 (tools/compiler/weights.cpp:72-105,
//          tools/runtime/formats.cpp:35-56), as smolvla_common.cpp:95-103
//          chains them for a W8 layer.
//   MXFP4: CanonicalMxfp4 (weights.cpp:39-70) over the codes and scale bytes
//          ReadMxfp4 reads (weights.cpp:120-138).
// One thread per (row, 32-element block): a row of the weight matrix is an
// output column of the layer, so thread (r, b) writes the 16 code bytes of
// column r % 8 of word (r / 8, b), its scale byte, and (column 0) the word's
// padding.
#include "hb_device.h"
#include "hb_internal.h"

namespace hb {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 32 nibbles (element k in the low 4 bits of n[k]) -> the 16 bytes of a WBUF
// column-block, element 2j in the low nibble of byte j.
__device__ __forceinline__ u32x4 PackNibbles(const uint8_t* n) {
  u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int k = 0; k < 32; ++k) v[k / 8] |= (uint32_t)(n[k] & 15u) << (4 * (k % 8));
  return v;
}

__device__ __forceinline__ void PutColumn(uint8_t* words, uint32_t row, uint32_t blk,
                                          uint32_t blocks, const u32x4& codes, uint32_t scale) {
  uint8_t* word = words + ((size_t)(row / 8) * blocks + blk) * kDdrWord;
  *reinterpret_cast<u32x4*>(word + (row % 8) * 16) = codes;
  word[128 + row % 8] = (uint8_t)scale;
  if (row % 8 == 0) *reinterpret_cast<uint2*>(word + 136) = uint2{0u, 0u};
}

// fp32 weights [rows][cols] -> the hi and lo W8 planes [out_rows / 8][blocks].
// Rows past `rows` (PadRows) and columns past `cols` (EncodeMxint8's
// padding to a whole block) are zeros: code 0, block exponent 0.  Inf or NaN
// sets *bad (the reference rejects them).
__global__ __launch_bounds__(256) void W8FromFp32Kernel(const float* w, uint32_t rows,
                                                        uint32_t cols, uint32_t out_rows,
                                                        uint32_t blocks, uint8_t* hi, uint8_t* lo,
                                                        uint32_t* bad_flag) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)out_rows * blocks) return;
  const uint32_t row = (uint32_t)(i / blocks), blk = (uint32_t)(i % blocks);
  uint32_t bits[32];
  uint32_t amax = 0;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const uint32_t col = blk * 32 + k;
    bits[k] = row < rows && col < cols ? __float_as_uint(w[(size_t)row * cols + col]) : 0u;
    amax = max(amax, bits[k] & 0x7FFFFFFFu);
  }
  const int32_t e = amax ? (int32_t)ExpField(amax) - 127 : 0;
  bool bad = false;
  uint8_t h[32], l[32];
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    const uint8_t q = (uint8_t)QuantizeInt8(bits[k], e, &bad);
    h[k] = q >> 4;
    l[k] = q & 15u;
  }
  PutColumn(hi, row, blk, blocks, PackNibbles(h), (uint32_t)(e + 127));
  PutColumn(lo, row, blk, blocks, PackNibbles(l), (uint32_t)(e + 127));
  if (bad) atomicOr(bad_flag, 1u);
}

// MXFP4 codes (one E2M1 code per byte, low nibble) [rows][cols] and E8M0
// scale bytes [rows][cols / 32] -> canonical WBUF words [out_rows / 8][blocks]:
// each block's codes rescaled so that its largest magnitude has E2M1
// exponent 2, the difference (and exponent_shift) moved into its exponent.
// A block of zeros keeps exponent 0; rows past `rows` are such blocks.  A
// code the rescale cannot represent, or an exponent outside E8M0, sets
// *bad (the reference rejects both).
__global__ __launch_bounds__(256) void Mxfp4CanonicalKernel(const uint8_t* codes,
                                                            const uint8_t* scales, uint32_t rows,
                                                            uint32_t cols, int32_t shift_in,
                                                            uint32_t out_rows, uint32_t blocks,
                                                            uint8_t* out, uint32_t* bad_flag) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (uint64_t)out_rows * blocks) return;
  const uint32_t row = (uint32_t)(i / blocks), blk = (uint32_t)(i % blocks);
  // E2M1 magnitudes in half units and their floor(log2) (weights.cpp's tables)
  constexpr uint32_t kHalf[8] = {0, 1, 2, 3, 4, 6, 8, 12};
  constexpr int32_t kFloorLog2[8] = {0, -1, 0, 0, 1, 1, 2, 2};
  uint8_t c[32];
  uint32_t top = 0;
#pragma unroll
  for (int k = 0; k < 32; ++k) {
    c[k] = row < rows ? codes[(size_t)row * cols + blk * 32 + k] : 0;
    top = max(top, (uint32_t)(c[k] & 7u));
  }
  bool bad = false;
  int32_t e = 0;
  if (top == 0) {  // the block stays zero codes (a -0 code included) with exponent 0
#pragma unroll
    for (int k = 0; k < 32; ++k) c[k] = 0;
  } else {
    e = (int32_t)scales[(size_t)row * blocks + blk] - 127 + kFloorLog2[top] - 2 + shift_in;
    const int32_t up = 2 - kFloorLog2[top];
#pragma unroll
    for (int k = 0; k < 32; ++k) {
      const uint32_t half = kHalf[c[k] & 7u] << up;
      uint32_t idx = 8;
#pragma unroll
      for (uint32_t j = 0; j < 8; ++j) idx = kHalf[j] == half ? j : idx;
      bad |= idx == 8;
      idx &= 7u;
      c[k] = (uint8_t)((idx != 0 && (c[k] & 8u)) ? (idx | 8u) : idx);
    }
    bad |= e < -127 || e > 127;
  }
  PutColumn(out, row, blk, blocks, PackNibbles(c), (uint32_t)(e + 127) & 0xFFu);
  if (bad) atomicOr(bad_flag, 1u);
}

}  // namespace

hipError_t LaunchW8FromFp32(const float* w, uint32_t rows, uint32_t cols, uint32_t out_rows,
                            uint8_t* hi, uint8_t* lo, uint32_t* bad_flag, hipStream_t stream) {
  const uint32_t blocks = (cols + 31) / 32;
  const uint64_t n = (uint64_t)out_rows * blocks;
  hipLaunchKernelGGL(W8FromFp32Kernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, stream, w,
                     rows, cols, out_rows, blocks, hi, lo, bad_flag);
  return hipGetLastError();
}

hipError_t LaunchMxfp4Canonical(const uint8_t* codes, const uint8_t* scales, uint32_t rows,
                                uint32_t cols, int32_t exponent_shift, uint32_t out_rows,
                                uint8_t* out, uint32_t* bad_flag, hipStream_t stream) {
  const uint32_t blocks = cols / 32;
  const uint64_t n = (uint64_t)out_rows * blocks;
  hipLaunchKernelGGL(Mxfp4CanonicalKernel, dim3((uint32_t)((n + 255) / 256)), dim3(256), 0, stream,
                     codes, scales, rows, cols, exponent_shift, out_rows, blocks, out, bad_flag);
  return hipGetLastError();
}

}  // namespace hb
