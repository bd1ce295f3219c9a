// GEMM kernels for gfx950: the hotarubi GEMM instruction (ISS images) and
// the linear layer it is emitted for (DDR words), both exact.
//
// Arithmetic (tools/iss/gemm_array.cpp:51-69, 99-110): per output and per
// 32-element K block, the block value s * 2^(ea + ew + SBIAS) with s the exact
// integer dot product, folded into an FP32 accumulator in block order.
//
// Matrix-core mapping.  Per K block the tile's operands are staged in LDS as
// bf16: A' = q * 2^(ea-127) (its E8M0 scale folded in) and W' = v, the
// unscaled weight value.  q (int8) and v (4-bit value) have at most 8
// significant bits, so A' and W' are exact bf16 values whenever the scale
// keeps A' normal.  One v_mfma_f32_16x16x32_bf16 with a zero accumulator then
// covers exactly one K block, and every product and every partial sum it
// forms is an integer multiple of 2^(ea-127) below 2^17 of that unit:
// all exactly representable, so the MFMA returns the exact block value up to
// W's scale.  The ordered fold is one fma per output and block,
// acc = fma(value, 2^(ew-127+SBIAS), acc): a single rounding of an exact sum
// (FTZ mode), which is the NPU's RNE add for normal operands; a -0 result
// can only appear where the NPU has +0 and is fixed once after the fold.
//
// The argument needs every scale byte of the tile in [70, 179] (exponents
// -57..52) and |initial C| < 2^126: then operands and products stay normal
// and the fold cannot overflow (steps <= 8192).  A tile that sees anything
// else recomputes itself with the integer routines of hb_fp32.h, so the
// result is bit-exact for every input.
//
// HB_LINEAR_FAST lets the MFMA accumulate (C = acc) instead of folding each
// block separately; that changes only the order of the FP32 additions.
#include "hb_device.h"
#include "hb_internal.h"

namespace hb {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;  // 4 waves
constexpr int kLdsRow = 40;    // bf16 per LDS row: 32 + 8 pad (80 B: conflict-free b128 reads)
#ifndef HB_CHUNK
#define HB_CHUNK 2
#endif
constexpr int kChunk = HB_CHUNK;  // K blocks per register prefetch chunk
constexpr uint32_t kSafeLo = 70, kSafeHi = 179;

// Tile geometry.  kBM x kBN outputs per workgroup; the 4 waves tile it as
// kWaveM x kWaveN with a kTM x kTN wave tile of 16x16 MFMA tiles.
template <int kBM, int kBN>
struct Tile {
  static constexpr int kTM = kBM >= 64 ? 64 : kBM;
  static constexpr int kWaveM = kBM / kTM;
  static constexpr int kWaveN = 4 / kWaveM;
  static constexpr int kTN = kBN / kWaveN;
  static constexpr int kTI = kTM / 16, kTJ = kTN / 16;
  static constexpr int kABytes = kBM * 32 / kThreads;  // A bytes a thread stages per block
  static constexpr int kWBytes = kBN * 16 / kThreads;  // W bytes a thread stages per block
  static constexpr int kA4 = kABytes / 4, kW4 = kWBytes / 4;
  static constexpr int kARowThreads = 32 / kABytes, kWColThreads = 16 / kWBytes;
  static_assert(kWaveM * kWaveN == 4 && kTN == 64, "wave tile is kTM x 64");
  static_assert(kABytes % 4 == 0 && kWBytes % 4 == 0, "whole dwords per thread");
};

struct Step {
  uint32_t p, l, b;  // piece, plane, block within the piece
};

// The step after s in fold order (pieces, planes, blocks), by selects only:
// the step loop stays one basic block.
__device__ __forceinline__ Step Next(const Step& s, const GemmArgs& g) {
  Step n;
  const bool wrap_b = s.b + 1 == g.piece_kb[s.p];
  const bool wrap_l = wrap_b && s.l + 1 == g.n_planes;
  n.b = wrap_b ? 0u : s.b + 1;
  n.l = wrap_l ? 0u : (wrap_b ? s.l + 1 : s.l);
  n.p = wrap_l ? s.p + 1 : s.p;
  return n;
}

template <bool kLinear>
__device__ __forceinline__ const uint8_t* AWord(const GemmArgs& g, const uint8_t* a, uint32_t q,
                                                uint32_t blk) {
  if (kLinear) return a + ((size_t)q * g.a_row + blk) * kDdrWord;
  return a + (size_t)((g.a_base + q * g.a_stride + blk) & (kAbufDepth - 1)) * kAbufWord;
}

template <bool kLinear>
__device__ __forceinline__ const uint8_t* WWord(const GemmArgs& g, const uint8_t* w, uint32_t grp,
                                                uint32_t blk) {
  if (kLinear) return w + ((size_t)grp * g.kb_total + blk) * kDdrWord;
  return w + (size_t)((g.w_base + grp * g.w_stride + blk) & (kWbufDepth - 1)) * kWbufWord;
}

// FP32 bits of the C element (row, col) of the tile's global index space.
template <bool kLinear>
__device__ __forceinline__ uint32_t* CElem(const GemmArgs& g, uint32_t* c, uint32_t row,
                                           uint32_t col) {
  if (kLinear) return c + (size_t)row * g.n + col;
  const uint32_t word = (g.c_base + (row >> 2) * g.groups + (col >> 3)) & (kFbufDepth - 1);
  return c + (size_t)word * 32 + (row & 3) * 8 + (col & 7);
}

// Which bytes of a K block a thread stages.  A: row r (token t of quad
// q0 + r/4), bytes [aofs, aofs + kABytes) of its 32; W: column col (lane cl
// of group g0 + col/8), bytes [wofs, wofs + kWBytes) of its 16.  In the
// 128-row tile, 8 consecutive lanes take 8 consecutive rows at the same
// byte offset, so their 16-byte LDS stores hit 8 distinct bank groups
// (80-byte rows: 80 r mod 128 is a permutation of the 16-byte slots).
template <class T>
struct Lane {
  uint32_t r, aofs, col, wofs;
  __device__ __forceinline__ Lane() {
    const uint32_t tid = threadIdx.x;
    if (T::kARowThreads == 2) {
      r = (tid & 7) + 8 * (tid >> 4);
      aofs = ((tid >> 3) & 1) * T::kABytes;
    } else {
      r = tid / T::kARowThreads;
      aofs = (tid % T::kARowThreads) * T::kABytes;
    }
    if (T::kWColThreads == 2) {
      col = (tid & 7) + 8 * (tid >> 4);
      wofs = ((tid >> 3) & 1) * T::kWBytes;
    } else {
      col = tid / T::kWColThreads;
      wofs = (tid % T::kWColThreads) * T::kWBytes;
    }
  }
};

// Raw operand bytes of one K block, as one thread stages them.  Loads are
// issued unconditionally: rows and columns past the edge of the layer read
// the last valid quad or group instead, which only feeds outputs that are
// never stored (rows of a GEMM depend on their own A row, columns on their
// own W column).  The load count per chunk is static, so the compiler waits
// on exactly the chunk being consumed while the next one is in flight.
template <int kA4, int kW4>
struct Staged {
  uint32_t a[kA4];
  uint32_t w[kW4];
  uint32_t sa, sw, plane;
  bool zero_a;  // a surplus step past the end: A stages as zeros
};

// Per-thread byte offsets of the staged bytes within a block's words
// (linear level: A word (q, blk) at (q * a_row + blk) * 144 and W word
// (grp, blk) at (grp * kb_total + blk) * 144, so the block index only moves
// a uniform base).
struct Offsets {
  uint32_t a, a_scale, w, w_scale;
};

template <bool kLinear, class T>
__device__ __forceinline__ Offsets ThreadOffsets(const GemmArgs& g, const Lane<T>& ln,
                                                 uint32_t q0, uint32_t g0) {
  const uint32_t quad = min(q0 + (ln.r >> 2), g.quads - 1), t = ln.r & 3;
  const uint32_t grp = min(g0 + (ln.col >> 3), g.groups - 1), cl = ln.col & 7;
  Offsets o;
  const uint32_t astride = kLinear ? g.a_row * kDdrWord : 0u;
  const uint32_t wstride = kLinear ? g.kb_total * kDdrWord : 0u;
  o.a = quad * astride + t * 32 + ln.aofs;
  o.a_scale = quad * astride + 128 + t;
  if (kLinear) {  // DDR words or panels (g.w_panels)
    const WLaneOff wo = WLane(g, grp * 8 + cl);
    o.w = wo.codes + ln.wofs;
    o.w_scale = wo.scale + wo.shift / 8;
  }
  (void)wstride;
  if (!kLinear) {  // keep the quad / group for the wrapping on-chip addresses
    o.a = (quad << 16) | (t * 32 + ln.aofs);
    o.a_scale = (quad << 16) | (128 + t);
    o.w = (grp << 16) | (cl * 16 + ln.wofs);
    o.w_scale = (grp << 16) | (128 + cl);
  }
  return o;
}

template <int kN>
__device__ __forceinline__ void LoadDwords(const uint8_t* p, uint32_t* out) {
  if (kN == 4) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = v[i];
  } else if (kN == 2) {
    const u32x2 v = *reinterpret_cast<const u32x2*>(p);
    out[0] = v[0];
    out[1] = v[1];
  } else {
#pragma unroll
    for (int i = 0; i < kN; ++i) out[i] = reinterpret_cast<const uint32_t*>(p)[i];
  }
}

template <bool kLinear, class T, class S>
__device__ __forceinline__ void LoadBlock(const GemmArgs& g, const uint8_t* a, const uint8_t* w0,
                                          const uint8_t* w1, const Offsets& o, const Step& s,
                                          S& st) {
  const uint32_t blk = g.piece_off[s.p] + s.b;
  st.plane = s.l;
  const uint8_t* w = s.l ? w1 : w0;
  if (kLinear) {
    const uint8_t* ab = a + (size_t)blk * kDdrWord;  // uniform
    LoadDwords<T::kA4>(ab + o.a, st.a);
    st.sa = ab[o.a_scale];
    LoadDwords<T::kW4>(w + WBlockCodes(g, blk) + o.w, st.w);  // uniform base + lane offset
    st.sw = w[WBlockScale(g, blk) + o.w_scale];
  } else {
    const uint8_t* aw = AWord<false>(g, a, o.a >> 16, blk);
    const uint8_t* ww = WWord<false>(g, w, o.w >> 16, blk);
    if (T::kA4 == 4) {  // ISS ABUF words are 132 B: only 4-byte aligned
#pragma unroll
      for (int i = 0; i < 4; ++i) st.a[i] = reinterpret_cast<const uint32_t*>(aw + (o.a & 0xFFFFu))[i];
    } else {
      LoadDwords<T::kA4>(aw + (o.a & 0xFFFFu), st.a);
    }
    st.sa = aw[o.a_scale & 0xFFFFu];
    LoadDwords<T::kW4>(ww + (o.w & 0xFFFFu), st.w);
    st.sw = ww[o.w_scale & 0xFFFFu];
  }
}

// 4 int8 -> 4 bf16 (2 dwords) scaled by fa = 2^(ea-127), exactly:
// (2^23 + q + 128) * fa - (2^23 + 128) * fa = q * fa, one rounding of an
// exact value.  The byte lands in a float's mantissa by v_perm_b32.
__device__ __forceinline__ void ConvertA4(uint32_t x, float fa, float fc, uint32_t* out) {
  const uint32_t xs = x ^ 0x80808080u;
  float f[4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
    f[i] = __builtin_fmaf(__uint_as_float(__builtin_amdgcn_perm(0x4B000000u, xs, 0x070C0C00u | i)),
                          fa, fc);
  out[0] = __builtin_amdgcn_perm(__float_as_uint(f[1]), __float_as_uint(f[0]), 0x07060302u);
  out[1] = __builtin_amdgcn_perm(__float_as_uint(f[3]), __float_as_uint(f[2]), 0x07060302u);
}

// bf16 bits of a small integer (exact).
__device__ __forceinline__ uint32_t Bf16OfInt(int32_t v) { return __float_as_uint((float)v) >> 16; }

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// 8 FP4 codes (one dword, low nibble first) -> 8 bf16 of 2 * E2M1 value,
// i.e. the reference's FP4 weight integers {0, +-1, ..., +-12}: one
// v_cvt_scalef32_pk_bf16_fp4 per byte (scale 2.0, exact).
__device__ __forceinline__ void ConvertFp4(uint32_t x, uint32_t* out) {
  out[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 0));
  out[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 1));
  out[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 2));
  out[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, 2.0f, 3));
}

// Stage one block into LDS: A scaled to bf16, W as unscaled bf16 weight
// integers, W scale bytes.  True if a scale byte is outside the window the
// matrix-core path is exact for.
template <class T, class S>
__device__ __forceinline__ bool StoreBlock(const S& st, const Lane<T>& ln, uint32_t mode,
                                           uint16_t* lds_a, uint16_t* lds_w, uint8_t* lds_ws,
                                           const uint32_t* lut) {
  const float fa = __uint_as_float(st.sa << 23);
  const float fc = -8388736.0f * fa;  // -(2^23 + 128) * fa
  uint32_t ab[2 * T::kA4];
#pragma unroll
  for (int i = 0; i < T::kA4; ++i) ConvertA4(st.a[i], fa, fc, ab + 2 * i);
#pragma unroll
  for (int i = 0; i < 2 * T::kA4; ++i) ab[i] = st.zero_a ? 0u : ab[i];
  uint32_t* da = reinterpret_cast<uint32_t*>(lds_a + ln.r * kLdsRow + ln.aofs);
  if (T::kA4 == 4) {
    reinterpret_cast<u32x4*>(da)[0] = u32x4{ab[0], ab[1], ab[2], ab[3]};
    reinterpret_cast<u32x4*>(da)[1] = u32x4{ab[4], ab[5], ab[6], ab[7]};
  } else {
    reinterpret_cast<u32x2*>(da)[0] = u32x2{ab[0], ab[1]};
  }
  uint32_t wb[4 * T::kW4];
  if (mode == kModeFp4) {
#pragma unroll
    for (int i = 0; i < T::kW4; ++i) ConvertFp4(st.w[i], wb + 4 * i);
  } else {
    const uint32_t* tab = lut + st.plane * 256;
#pragma unroll
    for (int i = 0; i < T::kW4; ++i)
#pragma unroll
      for (int m = 0; m < 4; ++m) wb[4 * i + m] = tab[(st.w[i] >> (8 * m)) & 0xFFu];
  }
  u32x4* dw = reinterpret_cast<u32x4*>(lds_w + ln.col * kLdsRow + ln.wofs * 2);
#pragma unroll
  for (int i = 0; i < T::kW4; ++i) dw[i] = u32x4{wb[4 * i], wb[4 * i + 1], wb[4 * i + 2], wb[4 * i + 3]};
  lds_ws[ln.col] = (uint8_t)st.sw;  // both threads of a column store the same byte
  return st.sa < kSafeLo || st.sa > kSafeHi || st.sw < kSafeLo || st.sw > kSafeHi;
}

// Exact integer recomputation of one output (the NPU's arithmetic verbatim).
template <bool kLinear>
__device__ __forceinline__ uint32_t SlowOutput(const GemmArgs& g, const uint8_t* a,
                                               const uint8_t* w0, const uint8_t* w1, uint32_t acc,
                                               uint32_t row, uint32_t col) {
  if (kLinear) return SlowLinear(g, a, w0, w1, acc, row, col);
  const uint32_t quad = row >> 2, t = row & 3, grp = col >> 3, cl = col & 7;
  for (uint32_t p = 0; p < g.n_pieces; ++p) {
    for (uint32_t l = 0; l < g.n_planes; ++l) {
      const uint32_t mode = g.modes[l];
      for (uint32_t b = 0; b < g.piece_kb[p]; ++b) {
        const uint32_t blk = g.piece_off[p] + b;
        const uint8_t* aw = AWord<kLinear>(g, a, quad, blk);
        const uint8_t* ww = WWord<kLinear>(g, l ? w1 : w0, grp, blk);
        int32_t sum = 0;
        for (uint32_t k = 0; k < 32; ++k) {
          const uint32_t byte = ww[cl * 16 + (k >> 1)];
          sum += (int32_t)(int8_t)aw[t * 32 + k] * WeightValue((k & 1) ? (byte >> 4) : byte, mode);
        }
        acc = AddBits(acc, BlockValue(sum, aw[128 + t], ww[128 + cl], mode));
      }
    }
  }
  return acc;
}

// The exact tile kernel.  Per K block: stage A (bf16, scaled) and W (bf16,
// unscaled) in LDS; per 16x16 tile one MFMA with a zero accumulator gives
// s * 2^(ea-127) exactly; the fold is acc = fma(that, 2^(ew-127+SBIAS), acc),
// a single rounding of an exact sum, which is the NPU's Fp32Add.  Operand
// loads run a chunk of kChunk blocks ahead of the compute.
template <bool kLinear, int kBM, int kBN>
__global__ __launch_bounds__(kThreads) void GemmTileKernel(GemmArgs g) {
  using T = Tile<kBM, kBN>;
  using S = Staged<T::kA4, T::kW4>;
  __shared__ __attribute__((aligned(16))) uint16_t lds_a[2][kBM * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint16_t lds_w[2][kBN * kLdsRow];
  __shared__ __attribute__((aligned(16))) uint8_t lds_ws[2][kBN];
  __shared__ uint32_t lut[2 * 256];
  __shared__ uint64_t lds_act[512];  // activation half of TBUF, for the epilogue
  __shared__ uint32_t lds_unsafe;

  const uint8_t* a = g.a;
  const uint8_t* w0 = g.w[0];
  const uint8_t* w1 = g.w[1];
  uint32_t* c = g.c;
  uint8_t* q_out = g.q_out;
  const TileId tile = LogicalTile(g.gx, g.gy, g.gz);
  const uint32_t z = kLinear ? tile.z : 0u;  // layer of a batched linear launch
  if (kLinear) {
    a += z * g.a_batch;
    w0 += z * g.w_batch;
    w1 += z * g.w_batch;
    c += z * g.c_batch;
    if (q_out) q_out += z * g.q_batch;
  }

  const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t wm = wave / T::kWaveN, wn = wave % T::kWaveN;
  const uint32_t row16 = lane & 15, kq = lane >> 4;
  const uint32_t q0 = tile.y * (kBM / 4), g0 = tile.x * (kBN / 8);
  const uint32_t row0 = q0 * 4, col0 = g0 * 8;

  const Lane<T> ln;
  const Offsets offs = ThreadOffsets<kLinear, T>(g, ln, q0, g0);
  if (tid == 0) lds_unsafe = 0;
  // byte -> two unscaled bf16 weight values (low nibble first), per plane
  for (uint32_t l = 0; l < g.n_planes; ++l) {
    const uint32_t mode = g.modes[l];
    lut[l * 256 + tid] = Bf16OfInt(WeightValue(tid & 15u, mode)) |
                         (Bf16OfInt(WeightValue(tid >> 4, mode)) << 16);
  }
  __syncthreads();  // the table and the cleared flag are visible to every wave

  // Output (i, j, v) of this lane: tile row wm*kTM + i*16 + kq*4 + v,
  // tile column wn*kTN + j*16 + row16 (16x16 MFMA accumulator layout).
  f32x4 acc[T::kTI][T::kTJ];
  bool unsafe = false;
#pragma unroll
  for (int i = 0; i < T::kTI; ++i)
#pragma unroll
    for (int j = 0; j < T::kTJ; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint32_t row = row0 + wm * T::kTM + i * 16 + kq * 4 + v;
        const uint32_t col = col0 + wn * T::kTN + j * 16 + row16;
        uint32_t init = 0;
        if (g.acc && (row >> 2) < g.quads && (col >> 3) < g.groups && (!kLinear || row < g.m)) {
          init = *CElem<kLinear>(g, c, row, col);
          unsafe |= ExpField(init) > 252u;
        }
        acc[i][j][v] = __uint_as_float(init);
      }

  // The step loop is one basic block: every wave runs every step (surplus
  // steps of the last iteration repeat the last block with A zeroed, adding
  // +0), the load cursor advances by selects, and scale bytes outside the
  // safe window are collected per thread and acted on once, after the loop.
  const uint32_t total = g.total_steps;
  Step ls{0, 0, 0};  // load cursor; stays on the last step once there
  uint32_t loaded = 0;
  // Loads issue in program order (the fences stop the scheduler from mixing
  // the two register sets), so the in-order load counter lets each compute
  // wait for exactly its own set.
  auto load_chunk = [&](S* set) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int b = 0; b < kChunk; ++b) {
      LoadBlock<kLinear, T>(g, a, w0, w1, offs, ls, set[b]);
      set[b].zero_a = loaded >= total;
      const Step nx = Next(ls, g);
      const bool adv = loaded + 1 < total;
      ls.p = adv ? nx.p : ls.p;
      ls.l = adv ? nx.l : ls.l;
      ls.b = adv ? nx.b : ls.b;
      ++loaded;
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto compute_chunk = [&](const S* set, uint32_t base) {
#pragma unroll
    for (int b = 0; b < kChunk; ++b) {
      const uint32_t buf = (base + b) & 1;
      unsafe |= StoreBlock<T>(set[b], ln, g.modes[set[b].plane], lds_a[buf], lds_w[buf],
                              lds_ws[buf], lut);
      __syncthreads();
      const int32_t wbias = ScaleBias(g.modes[set[b].plane]);
      bf16x8 af[T::kTI], bfr[T::kTJ];
      float fw[T::kTJ];
#pragma unroll
      for (int i = 0; i < T::kTI; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(
            &lds_a[buf][(wm * T::kTM + i * 16 + row16) * kLdsRow + kq * 8]);
#pragma unroll
      for (int j = 0; j < T::kTJ; ++j) {
        const uint32_t lc = wn * T::kTN + j * 16 + row16;
        bfr[j] = *reinterpret_cast<const bf16x8*>(&lds_w[buf][lc * kLdsRow + kq * 8]);
        fw[j] = __uint_as_float((uint32_t)((int32_t)lds_ws[buf][lc] + wbias) << 23);
      }
#pragma unroll
      for (int i = 0; i < T::kTI; ++i)
#pragma unroll
        for (int j = 0; j < T::kTJ; ++j) {
          const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
          const f32x4 bv = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], zero, 0, 0, 0);
#pragma unroll
          for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(bv[v], fw[j], acc[i][j][v]);
        }
      // Anchor the fold here: left free, the compiler sinks every step's
      // (pure) folds to the end of the iteration, keeping all the steps'
      // block values live at once.  The empty asm emits no instruction.
#pragma unroll
      for (int i = 0; i < T::kTI; ++i)
#pragma unroll
        for (int j = 0; j < T::kTJ; ++j) asm volatile("" : "+v"(acc[i][j]));
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Ping-pong over two register sets: each compute consumes one set while
  // the other set's loads are in flight.
  S set0[kChunk], set1[kChunk];
  load_chunk(set0);
  for (uint32_t base = 0; base < total; base += 2 * kChunk) {
    load_chunk(set1);
    compute_chunk(set0, base);
    load_chunk(set0);
    compute_chunk(set1, base + kChunk);
  }
  if (unsafe) lds_unsafe = 1;
  if (kLinear && g.tbuf != nullptr)
    for (uint32_t i = tid; i < 512; i += kThreads) lds_act[i] = g.tbuf[512 + i];
  __syncthreads();
  const bool slow = lds_unsafe != 0;

  // Results as FP32 bits in one 16-value register vector per row tile i
  // (element e = 4 * j + v).  i is unrolled and e, where a loop over it is
  // not, is a wave-uniform index into the vector, so nothing goes through
  // scratch memory.  The slow path recomputes the whole tile exactly.
  static_assert(T::kTJ == 4, "four 16-column tiles per wave");
  f32x16 res[T::kTI];
#pragma unroll
  for (int i = 0; i < T::kTI; ++i) {
    const f32x8 lo = __builtin_shufflevector(acc[i][0], acc[i][1], 0, 1, 2, 3, 4, 5, 6, 7);
    const f32x8 hi = __builtin_shufflevector(acc[i][2], acc[i][3], 0, 1, 2, 3, 4, 5, 6, 7);
    res[i] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t bits = __float_as_uint(res[i][e]);
      res[i][e] = __uint_as_float(bits == kSign ? 0u : bits);
    }
  }
  const uint32_t row_l = row0 + wm * T::kTM + kq * 4;
  const uint32_t col_l = col0 + wn * T::kTN + row16;
  if (slow) {
#pragma unroll
    for (int i = 0; i < T::kTI; ++i)
      for (uint32_t e = 0; e < 16; ++e) {
        const uint32_t row = row_l + i * 16 + (e & 3), col = col_l + (e >> 2) * 16;
        if ((row >> 2) >= g.quads || (col >> 3) >= g.groups) continue;
        uint32_t init = 0;
        if (g.acc && (!kLinear || row < g.m)) init = *CElem<kLinear>(g, c, row, col);
        res[i][e] = __uint_as_float(SlowOutput<kLinear>(g, a, w0, w1, init, row, col));
      }
  }
  if (kLinear && g.ws != nullptr) {  // deferred epilogue: the fold results, rows [0, 4*quads)
#pragma unroll
    for (int i = 0; i < T::kTI; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const uint32_t row = row_l + i * 16 + (e & 3), col = col_l + (e >> 2) * 16;
        if ((row >> 2) < g.quads && (col >> 3) < g.groups) g.ws[(size_t)row * g.n + col] = res[i][e];
      }
    return;
  }

  // Epilogue ops, op by op, in groups of two row tiles.  A group's operands
  // are loaded first, all at once (independent loads, one wait); the element
  // loop then only computes.
  if (kLinear) {
    constexpr int kGroup = T::kTI >= 2 ? 2 : 1;
    for (uint32_t o = 0; o < g.n_ops; ++o) {
      const uint32_t kind = g.op_kind[o], imm = g.op_imm[o];
      const bool has_x2 = kind == kEpAdd || kind == kEpActMul;
      const uint32_t* x2 = g.op_x2[o] + z * g.op_x2_batch[o];
      uint32_t pv[4] = {0u, 0u, 0u, 0u};
      if (kind == kEpAddP || kind == kEpMulP) {
        const uint32_t* v = g.op_vec[o] + z * g.op_vec_batch[o];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) pv[jj] = col_l + jj * 16 < g.n ? v[col_l + jj * 16] : 0u;
      }
#pragma unroll
      for (int i0 = 0; i0 < T::kTI; i0 += kGroup) {
        f32x16 xv[kGroup] = {};
        if (has_x2) {
#pragma unroll
          for (int ii = 0; ii < kGroup; ++ii)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
              const uint32_t row = row_l + (i0 + ii) * 16 + (e & 3), col = col_l + (e >> 2) * 16;
              xv[ii][e] = __uint_as_float(row < g.m && col < g.n ? x2[(size_t)row * g.n + col] : 0u);
            }
        }
#pragma unroll
        for (int ii = 0; ii < kGroup; ++ii) {
          const int i = i0 + ii;
          for (uint32_t e = 0; e < 16; ++e) {
            const uint32_t row = row_l + i * 16 + (e & 3), col = col_l + (e >> 2) * 16;
            if ((row >> 2) < g.quads && (col >> 3) < g.groups)
              res[i][e] = __uint_as_float(EpApply(kind, imm, __float_as_uint(res[i][e]),
                                                  __float_as_uint(xv[ii][e]), pv[e >> 2], lds_act));
          }
        }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < T::kTI; ++i)
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint32_t row = row_l + i * 16 + (e & 3), col = col_l + (e >> 2) * 16;
      const bool in_tile = (row >> 2) < g.quads && (col >> 3) < g.groups;
      if (in_tile && (!kLinear || (row < g.m && g.c != nullptr)))
        *CElem<kLinear>(g, c, row, col) = __float_as_uint(res[i][e]);
    }

  // MXINT8 requantize: one ABUF word per quad and 32 columns.  A quad is the
  // 4 accumulator rows (v) of one lane group (kq); a 32-column block is two
  // 16-column tiles (j, j+1) over the 16 lanes of the group.
  if (kLinear && q_out != nullptr) {
    const uint32_t nb = g.n >> 5;
#pragma unroll
    for (int i = 0; i < T::kTI; ++i) {
      const uint32_t quad = q0 + (wm * T::kTM + i * 16) / 4 + kq;
#pragma unroll
      for (int jb = 0; jb < T::kTJ; jb += 2) {
        const uint32_t blk = (col0 + wn * T::kTN + jb * 16) >> 5;
        uint32_t emax[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          emax[v] = RowMax16(max(ExpField(__float_as_uint(res[i][4 * jb + v])),
                                 ExpField(__float_as_uint(res[i][4 * jb + 4 + v]))));
        }
        if (quad < g.quads && blk < nb) {
          uint8_t* word = q_out + ((size_t)quad * nb + blk) * kDdrWord;
#pragma unroll
          for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int v = 0; v < 4; ++v)
              word[v * 32 + jj * 16 + row16] =
                  QuantizeElementHw(__float_as_uint(res[i][4 * (jb + jj) + v]), emax[v]);
          const uint32_t e_own =
              row16 == 0 ? emax[0] : row16 == 1 ? emax[1] : row16 == 2 ? emax[2] : emax[3];
          if (row16 < 4) word[128 + row16] = (uint8_t)ScaleByteOf(e_own);
          if (row16 >= 4) word[128 + row16] = 0;  // bytes 132..143
        }
      }
    }
  }
}

// An instruction whose output words wrap around FBUF (m/4 * n8 > 4096) writes
// some words more than once; with acc the later writers read what the earlier
// ones wrote.  This kernel keeps the reference's (g outer, q inner) order per
// FBUF word: one workgroup per word, one thread per element.
__global__ __launch_bounds__(32) void GemmAliasKernel(GemmArgs g) {
  const uint32_t total = g.quads * g.groups;
  const uint32_t i0 = blockIdx.x;
  uint32_t keys[16];
  uint32_t n = 0;
  for (uint32_t i = i0; i < total && n < 16; i += kFbufDepth)
    keys[n++] = (i % g.groups) * g.quads + i / g.groups;
  for (uint32_t x = 1; x < n; ++x) {  // ascending (g, q) order
    const uint32_t k = keys[x];
    uint32_t y = x;
    for (; y > 0 && keys[y - 1] > k; --y) keys[y] = keys[y - 1];
    keys[y] = k;
  }
  const uint32_t e = threadIdx.x, t = e >> 3, cl = e & 7;
  const uint32_t word = (g.c_base + i0) & (kFbufDepth - 1);
  uint32_t* elem = g.c + (size_t)word * 32 + e;
  const uint32_t mode = g.modes[0];
  for (uint32_t x = 0; x < n; ++x) {
    const uint32_t grp = keys[x] / g.quads, quad = keys[x] % g.quads;
    uint32_t acc = g.acc ? *elem : 0u;
    for (uint32_t b = 0; b < g.piece_kb[0]; ++b) {
      const uint8_t* aw = AWord<false>(g, g.a, quad, b);
      const uint8_t* ww = WWord<false>(g, g.w[0], grp, b);
      int32_t sum = 0;
      for (uint32_t k = 0; k < 32; ++k) {
        const uint32_t byte = ww[cl * 16 + (k >> 1)];
        sum += (int32_t)(int8_t)aw[t * 32 + k] * WeightValue((k & 1) ? (byte >> 4) : byte, mode);
      }
      acc = AddBits(acc, BlockValue(sum, aw[128 + t], ww[128 + cl], mode));
    }
    *elem = acc;
  }
}

}  // namespace

// 32 x 256 exact tiles for layers of at most 32 rows, and where the
// 128 x 128 grid (with the batch) leaves CUs idle while 32 x 256 tiles make
// more workgroups: each output's fold is sequential over K, so a small grid
// is parallel only across tiles (measured: SigLIP's 2048 x 768 x 3072 W8
// layer 235 -> 201 us, the SparseDrive-S head's layers at one frame 15-28%
// faster).
bool ExactShort(const GemmArgs& args, uint32_t batch) {
  if (args.quads * 4 <= 32) return true;
  const uint64_t tall = (uint64_t)((args.groups + 15) / 16) * ((args.quads + 31) / 32) * batch;
  const uint64_t shrt = (uint64_t)((args.groups + 31) / 32) * ((args.quads + 7) / 8) * batch;
  return tall < (uint64_t)DeviceCus() && shrt > tall;
}

template <bool kLinear>
hipError_t LaunchTiles(const GemmArgs& in, uint32_t batch, hipStream_t stream) {
  GemmArgs args = in;
  args.gz = batch;
  if (!kLinear ? args.quads * 4 <= 32 : ExactShort(args, batch)) {
    args.gx = (args.groups + 31) / 32;
    args.gy = (args.quads + 7) / 8;
    hipLaunchKernelGGL((GemmTileKernel<kLinear, 32, 256>), dim3(args.gx * args.gy * batch),
                       dim3(kThreads), 0, stream, args);
  } else {
    args.gx = (args.groups + 15) / 16;
    args.gy = (args.quads + 31) / 32;
    hipLaunchKernelGGL((GemmTileKernel<kLinear, 128, 128>), dim3(args.gx * args.gy * batch),
                       dim3(kThreads), 0, stream, args);
  }
  return hipGetLastError();
}

hipError_t LaunchGemmInstr(const GemmArgs& args, hipStream_t stream) {
  return LaunchTiles<false>(args, 1, stream);
}

hipError_t LaunchGemmInstrAliased(const GemmArgs& args, hipStream_t stream) {
  const uint32_t total = args.quads * args.groups;
  const uint32_t words = total < kFbufDepth ? total : kFbufDepth;
  hipLaunchKernelGGL(GemmAliasKernel, dim3(words), dim3(32), 0, stream, args);
  return hipGetLastError();
}

bool ExactShort(const GemmArgs& args, uint32_t batch);
void ExactGrid(const GemmArgs& args, uint32_t* gx, uint32_t* gy) {
  if (ExactShort(args, 1)) {
    *gx = (args.groups + 31) / 32;
    *gy = (args.quads + 7) / 8;
  } else {
    *gx = (args.groups + 15) / 16;
    *gy = (args.quads + 31) / 32;
  }
}

namespace {
// A single layer with fewer tiles than this spreads its work: K splits in
// fast mode (to about kTargetWorkgroups workgroups, at least kMinSplitSteps
// K-steps each) and the element-parallel deferred epilogue.  Measured on the
// SmolVLA chains (M = 141 and 1,600): 128 workgroups of at least 4 steps beat
// 256 of 2 by 9-13% (the split sums written and read again cost more than the
// parallelism gains); 32 workgroups, or no split, lost 50-70% at M = 141.
constexpr uint32_t kSmallGrid = 128, kTargetWorkgroups = 128, kMinSplitSteps = 4;
constexpr uint32_t kSplitMidRows = 1024, kSplitMidWork = 65536;
}  // namespace

hipError_t GrowWorkspace(Workspace& ws, size_t bytes, hipStream_t stream) {
  bytes += kSplitCounterBytes;
  if (ws.bytes >= bytes) return hipSuccess;
  // at least double, so a run of growing shapes retires few buffers
  size_t want = ws.bytes * 2 > bytes ? ws.bytes * 2 : bytes;
  want = (want + 0xFFFFF) & ~(size_t)0xFFFFF;
  if (ws.ptr != nullptr && ws.n_retired == sizeof ws.retired / sizeof ws.retired[0])
    return hipErrorOutOfMemory;  // (64 doublings: unreachable in practice)
  float* p = nullptr;
  hipError_t err = hipMalloc(&p, want);
  if (err != hipSuccess) return err;
  err = hipMemsetAsync(p, 0, kSplitCounterBytes, stream);  // the split counters start at zero
  if (err != hipSuccess) {
    (void)hipFree(p);
    return err;
  }
  if (ws.ptr != nullptr) ws.retired[ws.n_retired++] = ws.ptr;
  ws.ptr = p;
  ws.bytes = want;
  return hipSuccess;
}

void FreeWorkspace(Workspace& ws) {
  if (ws.ptr != nullptr) (void)hipFree(ws.ptr);
  for (uint32_t i = 0; i < ws.n_retired; ++i) (void)hipFree(ws.retired[i]);
  ws = Workspace{};
}

// MXFP8 E4M3 activations (one MXFP4 plane): in fast mode a layer of up to
// kSplitMidRows rows runs the single-launch split kernel with A straight
// into the FP8 x FP4 matrix cores; every other layer (exact mode, batches,
// more rows) is folded exactly per output by the epilogue kernel, one
// launch per layer (which meets the fast-mode tolerance too).
hipError_t LaunchFp8Linear(const GemmArgs& in, uint32_t batch, bool fast, hipStream_t stream) {
  GemmArgs args = in;
  args.ws = nullptr;
  args.splits = 1;
  args.split_steps = 0;
  if (fast && batch == 1 && args.quads * 4 <= kSplitMidRows) {
    SplitPlan(args);
    args.fast_ep = 1u;
    return LaunchSplitLinear(args, stream);
  }
  // batches of layers of up to 16 rows: the skinny kernel (the streaming
  // kernel's 128-row tiles would be mostly padding)
  if (fast && args.quads * 4 <= 16) {
    args.fast_ep = 1u;
    return LaunchLinearSkinny(args, batch, stream);
  }
  // batches and larger layers over weight panels (ops and the requantize
  // included): the streaming kernel, not the per-output exact fold below
  if (fast && StreamEligible(args)) {
    args.fast_ep = 1u;
    return LaunchStream(args, batch, stream);
  }
  args.fast_ep = 0u;
  for (uint32_t z = 0; z < batch; ++z) {
    GemmArgs one = args;
    one.a += z * args.a_batch;
    one.w[0] += z * args.w_batch;
    one.w[1] = one.w[0];
    one.c += z * args.c_batch;
    if (one.q_out != nullptr) one.q_out += z * args.q_batch;
    for (uint32_t o = 0; o < args.n_ops; ++o) {
      if (one.op_vec[o] != nullptr) one.op_vec[o] += z * args.op_vec_batch[o];
      if (one.op_x2[o] != nullptr) one.op_x2[o] += z * args.op_x2_batch[o];
    }
    one.a_batch = one.w_batch = one.c_batch = one.q_batch = 0;
    const hipError_t err = LaunchEpilogue(one, stream);
    if (err != hipSuccess) return err;
  }
  return hipSuccess;
}

hipError_t LaunchLinear(const GemmArgs& in, uint32_t batch, bool fast, Workspace& ws,
                        hipStream_t stream, FixedScratch* fixed) {
  // W8 panels: their own kernel, every shape and mode.
  if (in.w_fp6) return LaunchW8Linear(in, batch, fast, stream);
  if (in.a_fp8) return LaunchFp8Linear(in, batch, fast, stream);
  GemmArgs args = in;
  args.ws = nullptr;
  args.splits = 1;
  args.split_steps = 0;
  // Fast mode runs MXFP4 and W8 (hi, lo) on the block-scaled matrix cores;
  // any other plane list runs exactly (which meets the fast-mode tolerance).
  const bool fastk = fast && FastEligible(args);
  // A single small layer: one launch, K split over workgroups (the last
  // split of each tile finishes it).  Workspace: the counters, then the
  // partial sums.
  if (fastk && SplitEligible(args, batch)) {
    const size_t part = SplitPlan(args);
    args.fast_ep = 1u;
    if (part > 0) {
      float* base = nullptr;
      if (fixed != nullptr) {
        fixed->need = kSplitCounterBytes + part;
        if (fixed->need > fixed->bytes || fixed->ptr == nullptr) return hipErrorOutOfMemory;
        base = static_cast<float*>(fixed->ptr);
      } else {
        const hipError_t grown = GrowWorkspace(ws, part, stream);
        if (grown != hipSuccess) return grown;
        base = ws.ptr;
      }
      args.ws = base;
    }
    return LaunchSplitLinear(args, stream);
  }
  // Batched layers of up to 16 rows: split-K over the waves of one
  // workgroup, which holds every row.
  if (fastk && args.quads * 4 <= 16) return LaunchLinearSkinny(args, batch, stream);
  uint32_t gx, gy;
  if (fastk) FastGrid(args, batch, &gx, &gy, &args.tile_rows);
  else ExactGrid(args, &gx, &gy);
  args.gx = gx;
  args.gy = gy;
  const bool small = batch == 1 && gx * gy < kSmallGrid;
  // A layer of up to kSplitMidRows rows whose 128-row grid is small: the
  // single-launch split kernel's 32 x 32 tiles (enough workgroups, no
  // partial sums through memory, no second launch) instead of K splits of
  // 128-row tiles and the epilogue kernel, while rows x K blocks stays
  // within kSplitMidWork (measured, one layer per launch: 928 x 512 x 512
  // 7.3 against 16.1 us, 512 x 2560 x 960 18.1 against 25.9 us, 768 rows
  // even, 1024 x 2560 x 960 34.3 against 28.9 us).
  uint32_t blocks = 0;
  for (uint32_t p = 0; p < args.n_pieces; ++p) blocks += args.piece_kb[p];
  if (small && fastk && args.quads * 4 <= kSplitMidRows &&
      args.quads * 4 * blocks <= kSplitMidWork) {
    SplitPlan(args);
    args.fast_ep = 1u;
    return LaunchSplitLinear(args, stream);
  }
  args.fast_ep = fastk ? 1u : 0u;
  // Over panels the streaming kernel takes plain batched layers (and
  // MXFP8); a plain single layer takes the panel kernel, whose 8 waves per
  // CU hide more latency where a workgroup has one or two tiles (measured,
  // one layer per launch: 1,600 x 2,048 x 736 24.0 -> 16.9 us, 4,512 x
  // 2,560 x 960 48.7 -> 36.2 us, 14,848 x 256 x 1,024 26.6 -> 18.6 us,
  // 67,584 x 64 x 576 47.5 -> 40.9 us).  Layers with ops or the requantize
  // stay on the tile kernel: its epilogue runs on 16 waves per CU, the
  // streaming kernel's on 4 (measured on the SparseDrive backbone's layers,
  // e.g. 67,584 x 256 x 128 with bias, ReLU and the requantize: 55 against
  // 139 us).
  if (fastk && !small && StreamEligible(args) && (batch > 1 || args.a_fp8))
    return LaunchStream(args, batch, stream);
  if (fastk && !small && PanelEligible(args)) return LaunchPanel(args, batch, stream);
  if (small && fastk) {
    // as many splits as fit in one round of kTargetWorkgroups workgroups
    uint32_t nblocks = 0;
    for (uint32_t p = 0; p < args.n_pieces; ++p) nblocks += args.piece_kb[p];
    const uint32_t steps = (nblocks + 1) / 2;
    const uint32_t want = kTargetWorkgroups > gx * gy ? kTargetWorkgroups / (gx * gy) : 1u;
    uint32_t per = (steps + want - 1) / want;
    per = per < kMinSplitSteps ? kMinSplitSteps : per;
    args.splits = (steps + per - 1) / per;
    args.split_steps = per;
  }
  // The exact kernels' epilogue arithmetic is spread over the elements of a
  // small layer; the fast kernels finish an unsplit tile in place.
  const bool defer = small && (args.splits > 1 || (!fastk && (args.n_ops > 0 || args.q_out != nullptr)));
  if (!defer) return fastk ? LaunchLinearFast(args, batch, stream) : LaunchTiles<true>(args, batch, stream);

  // (the partial sums start after the split counters)
  if (fixed != nullptr) {  // no allocation: the caller's buffer, or an error
    fixed->need = kSplitCounterBytes + WorkspaceBytes(args);
    if (fixed->need > fixed->bytes || fixed->ptr == nullptr) return hipErrorOutOfMemory;
    args.ws = static_cast<float*>(fixed->ptr) + kSplitCounterBytes / sizeof(float);
  } else {
    const hipError_t grown = GrowWorkspace(ws, WorkspaceBytes(args), stream);
    if (grown != hipSuccess) return grown;
    args.ws = ws.ptr + kSplitCounterBytes / sizeof(float);
  }
  const hipError_t err = fastk ? LaunchLinearFast(args, args.splits, stream)  // z = split
                             : LaunchTiles<true>(args, 1, stream);
  if (err != hipSuccess) return err;
  return LaunchEpilogue(args, stream);
}

}  // namespace hb
