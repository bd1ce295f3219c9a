// C ABI of the hotarubi GEMM backend (include/hotarubi_gpu.h): contexts,
// device images of the on-chip memories, command validation and decoding,
// and the launches.  Everything computed here is bookkeeping on command
// fields; all arithmetic on operand data runs in the HIP kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>
#include <new>
#include <string>
#include <vector>

#include "hb_fp32.h"
#include "hb_internal.h"

struct hb_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  uint32_t* d_flag = nullptr;  // device flag word for hb_encode_mxint8
  hb::Workspace ws;            // split partials / deferred epilogue inputs
};

// DDR image (DdrImage, tools/compiler/ddr_image.cpp): regions in order of
// first placement, an index by name, the end of the last placed region.
struct hb_image {
  hb_ctx* ctx = nullptr;    // null: bookkeeping only
  uint8_t* bytes = nullptr;  // device memory, `capacity` bytes
  uint64_t capacity = 0, end = 0;
  bool reuse = false;
  std::vector<std::pair<std::string, std::pair<uint64_t, uint64_t>>> regions;  // offset, size
  std::map<std::string, size_t, std::less<>> index;
};

struct hb_onchip {
  hb_ctx* ctx = nullptr;
  uint8_t* abuf = nullptr;
  uint8_t* wbuf = nullptr;
  uint32_t* fbuf = nullptr;
  uint32_t* pbuf = nullptr;
  uint64_t* tbuf = nullptr;
  uint32_t* temp = nullptr;  // one VEC pass: up to 511 quads x 255 words x 32 values
};

// Scratch of hb_linear_noalloc_async: one array per device (the code
// object's copy on that device), never freed.  In host code `scratch` only
// names the symbol; its device address comes from hipGetSymbolAddress.
static __device__ __align__(256) uint8_t scratch[HB_NOALLOC_SCRATCH_BYTES];

namespace {

thread_local std::string g_error;

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch`, per device

int Fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int HipFail(hipError_t err, const char* what) {
  return Fail(HB_EDEVICE, "%s: %s", what, hipGetErrorString(err));
}

#define HB_HIP(call)                                  \
  do {                                                \
    hipError_t e_ = (call);                           \
    if (e_ != hipSuccess) return HipFail(e_, #call);  \
  } while (0)

// The scratch array's address on `device` (the current device), looked up
// once per device.
int ScratchSetUp(int device) {
  if (device < 0 || device >= kMaxDevices) return Fail(HB_EINVAL, "device %d", device);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[device] != nullptr) return HB_OK;
  void* p = nullptr;
  const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (err != hipSuccess) return HipFail(err, "scratch address");
  if (p == nullptr) return Fail(HB_EDEVICE, "scratch address is null");
  // the split kernel's tile counters start at zero (each launch puts back
  // what it used)
  HB_HIP(hipMemset(p, 0, hb::kSplitCounterBytes));
  g_scratch_ptr[device] = p;
  return HB_OK;
}

constexpr uint32_t kVecTempWords = 511u * 255u;

struct MemInfo {
  uint32_t depth, word;
};

MemInfo Info(int mem) {
  switch (mem) {
    case HB_MEM_ABUF: return {HB_ABUF_DEPTH, HB_ABUF_WORD_BYTES};
    case HB_MEM_WBUF: return {HB_WBUF_DEPTH, HB_WBUF_WORD_BYTES};
    case HB_MEM_FBUF: return {HB_FBUF_DEPTH, HB_FBUF_WORD_BYTES};
    case HB_MEM_PBUF: return {HB_PBUF_DEPTH, HB_PBUF_WORD_BYTES};
    case HB_MEM_TBUF: return {HB_TBUF_DEPTH, HB_TBUF_WORD_BYTES};
  }
  return {0, 0};
}

uint8_t* Image(hb_onchip* o, int mem) {
  switch (mem) {
    case HB_MEM_ABUF: return o->abuf;
    case HB_MEM_WBUF: return o->wbuf;
    case HB_MEM_FBUF: return reinterpret_cast<uint8_t*>(o->fbuf);
    case HB_MEM_PBUF: return reinterpret_cast<uint8_t*>(o->pbuf);
    case HB_MEM_TBUF: return reinterpret_cast<uint8_t*>(o->tbuf);
  }
  return nullptr;
}

// Preconditions of ExecuteGemm (tools/iss/gemm_array.cpp:113-119), with the
// reference's messages.
int CheckGemm(const hb_gemm_cmd* c) {
  if (!(c->m >= 32 && c->m <= 992 && c->m % 32 == 0))
    return Fail(HB_EBADCMD, "GEMM m = %u is not a multiple of 32 from 32 to 992", c->m);
  if (!(c->kb >= 1 && c->kb <= c->a_stride))
    return Fail(HB_EBADCMD, "GEMM kb = %u is not in [1, a_stride = %u]", c->kb, c->a_stride);
  if (c->n8 < 1) return Fail(HB_EBADCMD, "GEMM n8 = 0");
  // The instruction's n8 field is 8 bits wide (isa.hpp:83), so a decoded
  // command never exceeds 255.  The aliasing kernel relies on it: with m <= 992
  // an FBUF word then has at most ceil(248 * 255 / 4096) = 16 writers.
  if (c->n8 > 255)
    return Fail(HB_EINVAL, "GEMM n8 = %u does not fit the instruction's 8-bit field", c->n8);
  return HB_OK;
}

uint32_t Field(const uint8_t w[16], uint32_t lsb, uint32_t width) {
  uint64_t lo = 0, hi = 0;
  for (int i = 7; i >= 0; --i) lo = (lo << 8) | w[i];
  for (int i = 15; i >= 8; --i) hi = (hi << 8) | w[i];
  uint64_t v;
  if (lsb >= 64) v = hi >> (lsb - 64);
  else if (lsb == 0) v = lo;
  else v = (lo >> lsb) | (hi << (64 - lsb));
  return (uint32_t)(v & ((1ull << width) - 1ull));
}

void SetField(uint8_t w[16], uint32_t lsb, uint32_t width, uint32_t value) {
  for (uint32_t i = 0; i < width; ++i) {
    const uint32_t bit = lsb + i;
    const uint8_t mask = (uint8_t)(1u << (bit & 7));
    if ((value >> i) & 1u) w[bit >> 3] |= mask;
    else w[bit >> 3] &= (uint8_t)~mask;
  }
}

int Enter(hb_ctx* ctx) {
  if (!ctx) return Fail(HB_EINVAL, "null context");
  HB_HIP(hipSetDevice(ctx->device));
  return HB_OK;
}

hb::GemmArgs InstrArgs(const hb_gemm_cmd* cmd, hb_onchip* o) {
  hb::GemmArgs g;
  std::memset(&g, 0, sizeof g);
  g.a = o->abuf;
  g.w[0] = o->wbuf;
  g.w[1] = o->wbuf;
  g.c = o->fbuf;
  g.quads = cmd->m / 4;
  g.groups = cmd->n8;
  g.m = cmd->m;
  g.n = cmd->n8 * 8;
  g.a_base = cmd->a_base;
  g.a_stride = cmd->a_stride;
  g.w_base = cmd->w_base;
  g.w_stride = cmd->w_stride;
  g.c_base = cmd->c_base;
  g.n_pieces = 1;
  g.piece_off[0] = 0;
  g.piece_kb[0] = cmd->kb;
  g.n_planes = 1;
  g.modes[0] = hb::DecodeMode(cmd->wmode);
  g.total_steps = cmd->kb;
  g.acc = cmd->acc ? 1u : 0u;
  return g;
}

int GemmExec(hb_ctx* ctx, const hb_gemm_cmd* cmd, hb_onchip* o, bool sync) {
  if (int rc = Enter(ctx)) return rc;
  if (!cmd || !o) return Fail(HB_EINVAL, "null argument");
  if (int rc = CheckGemm(cmd)) return rc;
  const hb::GemmArgs g = InstrArgs(cmd, o);
  const uint64_t words = (uint64_t)g.quads * g.groups;
  hipError_t err = words <= hb::kFbufDepth ? hb::LaunchGemmInstr(g, ctx->stream)
                                           : hb::LaunchGemmInstrAliased(g, ctx->stream);
  if (err != hipSuccess) return HipFail(err, "GEMM launch");
  if (sync) HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

// ---- VEC: the passes of library entries 0-9 (tools/compiler/vec_rom.cpp:
// 63-70 Whole(), 214-237 Activation(), 314-349 Program()) ----

enum { kRSrc = 1, kRSrc2 = 2, kRDst = 3, kRImm = 8 };

struct PassSpec {
  uint32_t rx, rx2, rd;  // registers
  uint32_t c0, b, act, po, pv, rowvec, rimm;
  bool final_;
};

int LibraryPasses(uint32_t entry, PassSpec* out) {
  PassSpec p{kRSrc, 0, kRDst, 0, 0, 0, 0, 0, 0, 0, true};
  switch (entry) {
    case 0: p.rx2 = kRSrc2; p.c0 = 1; break;               // ADD
    case 1: p.rx2 = kRSrc2; p.b = 1; break;                // MUL
    case 2: p.rx2 = kRSrc2; p.po = 1; p.pv = 1; break;     // MAX
    case 3: p.rowvec = 1; p.c0 = 2; break;                 // ADDP
    case 4: p.rowvec = 1; p.b = 2; break;                  // MULP
    case 5: p.rimm = kRImm; p.b = 3; break;                // SCALE
    case 6: break;                                         // COPY
    case 7: p.po = 1; break;                               // RELU
    case 8:
    case 9: {                                              // ACT, ACT_MUL
      PassSpec sigma{kRSrc, 0, kRImm, 0, 0, 1, 0, 0, 0, 0, false};
      PassSpec gate{kRSrc, kRImm, kRDst, 0, 1, 0, 2, 0, 0, 0, true};
      out[0] = sigma;
      if (entry == 8) {
        out[1] = gate;
        return 2;
      }
      gate.rd = kRImm;
      gate.final_ = false;
      out[1] = gate;
      out[2] = PassSpec{kRImm, kRSrc2, kRDst, 0, 1, 0, 0, 0, 0, 0, true};
      return 3;
    }
    default: return 0;
  }
  out[0] = p;
  return 1;
}

// The failure checks of RunPass/RunQuads/RunWord/Store (vec_engine.cpp:
// 252-460) in program order, on addresses only.
int CheckPass(const hb::VecPass& p, const PassSpec& s) {
  if (p.quads == 0 || p.words == 0)
    return Fail(HB_EBADCMD, "a PASS has %u quads and %u words", p.quads, p.words);
  const uint32_t total = p.quads * p.words;
  if (!p.to_abuf) {
    std::vector<uint8_t> written(hb::kFbufDepth, 0);
    for (uint32_t i = 0; i < total; ++i) {
      const uint32_t xa = (p.src + i) & (hb::kFbufDepth - 1);
      if (written[xa]) return Fail(HB_EBADCMD, "a PASS reads FBUF word %u after writing it", xa);
      if (p.x2_en) {
        const uint32_t x2a = (p.src2 + i) & (hb::kFbufDepth - 1);
        if (written[x2a])
          return Fail(HB_EBADCMD, "a PASS reads FBUF word %u after writing it", x2a);
      }
      written[(p.d + i) & (hb::kFbufDepth - 1)] = 1;
    }
  } else if (p.n8 % 4 != 0) {
    if (p.quads >= 2) return Fail(HB_EBADCMD, "quantized word 0 arrives out of order");
    return Fail(HB_EBADCMD, "a PASS ends inside a block of 4 quantized words");
  }
  (void)s;
  return HB_OK;
}

uint32_t HostNegate(uint32_t b) { return (b & 0x7FFFFFFFu) == 0 ? 0u : b ^ 0x80000000u; }

// CountReciprocal (tools/iss/scalar.cpp:44-52, 64-69) for the Smem kRn
// step of the norm programs.
uint32_t HostCountReciprocal(uint32_t count) {
  const uint32_t n = count & 0x3FFFu;
  const int top = n == 0 ? 0 : hb::BitWidth32(n) - 1;
  const uint32_t x = ((uint32_t)(127 + top) << 23) | ((n << (23 - top)) & 0x7FFFFFu);
  uint32_t y = 0x7EF311C7u - x;
  for (int i = 0; i < 4; ++i) y = hb::MulBits(y, hb::AddBits(0x40000000u, HostNegate(hb::MulBits(x, y))));
  return y;
}

// Row programs (SOFTMAX, LAYERNORM, RMSNORM): the engine's failures in its
// order (pairs of quads pass by pass, vec_rom.cpp:84-131 with two row
// contexts; vec_engine.cpp:264-266, 383-387, 282-283), then the launch: the
// quads in parallel where none touches a word another writes, else in the
// engine's order.
int VecRows(hb_ctx* ctx, const hb_vec_cmd* cmd, hb_onchip* o) {
  hb::VecRowArgs a{};
  a.entry = cmd->entry;
  a.quantize = cmd->quantize ? 1u : 0u;
  a.rows_q = cmd->rows_q & 0x1FFu;
  a.n8 = cmd->n8 & 0xFFu;
  a.src = cmd->src & 0xFFFu;
  a.dst = cmd->dst & 0x1FFFu;
  a.pbase = cmd->p_base & 0x1FFu;
  a.aux = cmd->aux & 0x7FFu;
  a.imm = cmd->imm;
  a.quarter = a.n8 >> 2;
  a.dst_step = a.n8 - (a.n8 - a.quarter) * a.quantize;
  a.scratch = a.entry == hb::kRowSoftmax ? a.imm : (cmd->src2 & 0xFFFu);
  a.rn = HostCountReciprocal(a.aux);
  const uint32_t fmask = hb::kFbufDepth - 1, amask = hb::kAbufDepth - 1;
  std::vector<uint8_t> written(hb::kFbufDepth);
  hb::RowPassSpan spans[2][5];
  const uint32_t groups = a.rows_q >> 1, tail = a.rows_q & 1u;
  for (uint32_t g = 0; g <= groups; ++g) {
    const uint32_t slots = g < groups ? 2u : tail;
    int n = 0;
    for (uint32_t k = 0; k < slots; ++k) n = hb::RowProgramSpans(a, 2 * g + k, spans[k]);
    for (int i = 0; i < n; ++i)
      for (uint32_t k = 0; k < slots; ++k) {
        const hb::RowPassSpan& sp = spans[k][i];
        if (a.n8 == 0) return Fail(HB_EBADCMD, "a PASS has 1 quads and 0 words");
        std::fill(written.begin(), written.end(), 0);
        const bool fbuf_store = sp.writes && !(sp.final_ && a.quantize);
        for (uint32_t w = 0; w < a.n8; ++w) {
          const uint32_t xa = (sp.src + w) & fmask;
          if (written[xa]) return Fail(HB_EBADCMD, "a PASS reads FBUF word %u after writing it", xa);
          if (fbuf_store) written[(sp.dst + w) & fmask] = 1;
        }
        if (sp.final_ && a.quantize && a.n8 % 4 != 0)
          return Fail(HB_EBADCMD, "a PASS ends inside a block of 4 quantized words");
      }
  }
  // The quads run in parallel only if no word one quad writes is touched by
  // another.
  bool serial = false;
  std::vector<int32_t> owner(hb::kFbufDepth, -1), abuf_owner(hb::kAbufDepth, -1);
  for (uint32_t q = 0; q < a.rows_q && !serial; ++q) {
    hb::RowPassSpan sp[5];
    const int n = hb::RowProgramSpans(a, q, sp);
    for (int i = 0; i < n; ++i) {
      if (!sp[i].writes) continue;
      if (sp[i].final_ && a.quantize) {
        for (uint32_t b = 0; b < a.n8 / 4; ++b) {
          int32_t& ow = abuf_owner[((sp[i].dst & amask) + b) & amask];
          serial |= ow >= 0 && ow != (int32_t)q;
          ow = (int32_t)q;
        }
        continue;
      }
      for (uint32_t w = 0; w < a.n8; ++w) {
        int32_t& ow = owner[(sp[i].dst + w) & fmask];
        serial |= ow >= 0 && ow != (int32_t)q;
        ow = (int32_t)q;
      }
    }
  }
  for (uint32_t q = 0; q < a.rows_q && !serial; ++q) {
    hb::RowPassSpan sp[5];
    const int n = hb::RowProgramSpans(a, q, sp);
    for (int i = 0; i < n; ++i)
      for (uint32_t w = 0; w < a.n8; ++w) {
        const int32_t ow = owner[(sp[i].src + w) & fmask];
        serial |= ow >= 0 && ow != (int32_t)q;
      }
  }
  hipError_t err = hb::LaunchVecRows(a, o->abuf, o->fbuf, o->pbuf, o->tbuf, ctx->stream, serial);
  if (err != hipSuccess) return HipFail(err, "VEC row program launch");
  HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

int Rows(hb_ctx* ctx, const hb_rows_desc* d, bool sync) {
  if (int rc = Enter(ctx)) return rc;
  if (!d) return Fail(HB_EINVAL, "null descriptor");
  if (d->entry != HB_ROWS_SOFTMAX && d->entry != HB_ROWS_LAYERNORM && d->entry != HB_ROWS_RMSNORM)
    return Fail(HB_EUNSUPPORTED, "row program %u (12 SOFTMAX, 22 LAYERNORM, 34 RMSNORM)", d->entry);
  if (d->rows < 1 || d->cols < 8 || d->cols % 8 != 0 || d->cols > 2040)
    return Fail(HB_EINVAL, "rows = %u, cols = %u: need rows >= 1, cols a multiple of 8 up to 2040",
                d->rows, d->cols);
  if (!d->x || (d->y == nullptr) == (d->q_out == nullptr))
    return Fail(HB_EINVAL, "need x and exactly one of y, q_out");
  if (d->q_out && d->cols % 32 != 0) return Fail(HB_EINVAL, "q_out needs cols %% 32 == 0");
  // fp32 rows and vectors are read and written as words, the DDR words'
  // codes as dwords
  const void* bufs[] = {d->x, d->y, d->q_out, d->gamma, d->beta};
  for (const void* ptr : bufs)
    if (reinterpret_cast<uintptr_t>(ptr) % 4 != 0)
      return Fail(HB_EINVAL, "row buffers must be 4-byte aligned");
  if (d->entry != HB_ROWS_SOFTMAX && !d->gamma) return Fail(HB_EINVAL, "the norm needs gamma");
  if (d->entry == HB_ROWS_LAYERNORM && !d->beta) return Fail(HB_EINVAL, "LAYERNORM needs beta");
  // the program reads beta from PBUF word p_base + n8/4: a separate row only
  // when gamma fills whole words
  if (d->entry == HB_ROWS_LAYERNORM && d->cols % 32 != 0)
    return Fail(HB_EINVAL, "LAYERNORM needs cols %% 32 == 0");
  if (d->entry == HB_ROWS_SOFTMAX && !d->tbuf) return Fail(HB_EINVAL, "SOFTMAX needs TBUF");
  if ((d->rows + 3) / 4 > 0x7FFFFFFFu) return Fail(HB_EINVAL, "too many rows");
  hb::VecRowArgs a{};
  a.entry = d->entry;
  a.quantize = d->q_out ? 1u : 0u;
  a.rows_q = (d->rows + 3) / 4;
  a.n8 = d->cols / 8;
  a.quarter = a.n8 >> 2;
  a.aux = d->aux & 0x7FFu;  // the command field's width
  a.imm = d->imm;
  a.rn = HostCountReciprocal(a.aux);
  hb::VecRowDdr r{};
  r.x = reinterpret_cast<const uint32_t*>(d->x);
  r.gamma = reinterpret_cast<const uint32_t*>(d->gamma);
  r.beta = reinterpret_cast<const uint32_t*>(d->beta);
  r.y = reinterpret_cast<uint32_t*>(d->y);
  r.q_out = static_cast<uint8_t*>(d->q_out);
  r.rows = d->rows;
  r.cols = d->cols;
  hipError_t err = hb::LaunchRowsDdr(a, r, d->tbuf, ctx->stream);
  if (err != hipSuccess) return HipFail(err, "row program launch");
  if (sync) HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

int VecExec(hb_ctx* ctx, const hb_vec_cmd* cmd, hb_onchip* o) {
  if (int rc = Enter(ctx)) return rc;
  if (!cmd || !o) return Fail(HB_EINVAL, "null argument");
  if (cmd->entry == hb::kRowSoftmax || cmd->entry == hb::kRowLayerNorm ||
      cmd->entry == hb::kRowRmsNorm)
    return VecRows(ctx, cmd, o);
  PassSpec specs[3];
  const int n = LibraryPasses(cmd->entry, specs);
  if (n == 0)
    return Fail(HB_EUNSUPPORTED,
                "VEC library entry %u is not supported (0-9, 12 SOFTMAX, 22 LAYERNORM, 34 RMSNORM)",
                cmd->entry);
  // VecEngine::Initialize (vec_engine.cpp:227-239): operand field widths.
  uint32_t reg[16] = {0};
  reg[kRSrc] = cmd->src & 0xFFFu;
  reg[kRSrc2] = cmd->src2 & 0xFFFu;
  reg[kRDst] = cmd->dst & 0x1FFFu;
  reg[kRImm] = cmd->imm;
  const uint32_t rows_q = cmd->rows_q & 0x1FFu, n8 = cmd->n8 & 0xFFu;
  const uint32_t p_base = cmd->p_base & 0x1FFu;
  hb::VecPass passes[3];
  for (int i = 0; i < n; ++i) {
    const PassSpec& s = specs[i];
    hb::VecPass& p = passes[i];
    std::memset(&p, 0, sizeof p);
    p.src = reg[s.rx] & 0xFFFu;
    p.src2 = reg[s.rx2] & 0xFFFu;
    p.x2_en = s.rx2 != 0;
    p.d = reg[s.rd];
    p.c0 = s.c0;
    p.b = s.b;
    p.act = s.act;
    p.po = s.po;
    p.pv = s.pv;
    p.imm = reg[s.rimm];
    p.pb = p_base;
    p.quads = rows_q;
    p.words = n8;
    p.n8 = n8;
    p.to_abuf = s.final_ && cmd->quantize;
    p.d = p.to_abuf ? (p.d & (hb::kAbufDepth - 1)) : (p.d & (hb::kFbufDepth - 1));
    if (int rc = CheckPass(p, s)) return rc;
  }
  for (int i = 0; i < n; ++i) {
    hipError_t err =
        hb::LaunchVecPass(passes[i], o->abuf, o->fbuf, o->pbuf, o->tbuf, o->temp, ctx->stream);
    if (err != hipSuccess) return HipFail(err, "VEC launch");
  }
  HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

// ---- linear ----

bool ValidMode(uint32_t m) { return m <= 2; }

// Word offset of piece p's A words from its W blocks (a_word - kb_offset;
// 0 without a_stride).  The kernels address A by the W block index: a layer
// whose pieces share one offset runs with A's base moved by it.
int64_t PieceShift(const hb_linear_desc& d, uint32_t p) {
  return d.a_stride ? (int64_t)d.pieces[p].a_word - (int64_t)d.pieces[p].kb_offset : 0;
}

// Validates a descriptor and fills the kernel arguments.  *mixed is set when
// its pieces' A words sit at different offsets from their W blocks (see
// LinearChain).
int LinearArgs(const hb_linear_desc* d, hb::GemmArgs* g, bool* mixed) {
  if (!d) return Fail(HB_EINVAL, "null descriptor");
  if (d->m < 1 || d->n < 8 || d->n % 8 != 0 || d->kb_total < 1)
    return Fail(HB_EINVAL, "linear m = %u, n = %u, kb_total = %u: need m >= 1, n %% 8 == 0",
                d->m, d->n, d->kb_total);
  if (d->n_planes < 1 || d->n_planes > 2) return Fail(HB_EINVAL, "n_planes = %u", d->n_planes);
  for (uint32_t l = 0; l < d->n_planes; ++l)
    if (!ValidMode(d->modes[l]) || !d->w[l])
      return Fail(HB_EINVAL, "plane %u: mode %u / weights missing", l, d->modes[l]);
  if (d->n_pieces < 1 || d->n_pieces > HB_MAX_PIECES)
    return Fail(HB_EINVAL, "n_pieces = %u", d->n_pieces);
  uint64_t steps = 0;
  for (uint32_t p = 0; p < d->n_pieces; ++p) {
    const hb_piece& pc = d->pieces[p];
    if (pc.kb < 1 || (uint64_t)pc.kb_offset + pc.kb > d->kb_total)
      return Fail(HB_EINVAL, "piece %u [%u, +%u) is outside %u blocks", p, pc.kb_offset, pc.kb,
                  d->kb_total);
    steps += (uint64_t)pc.kb * d->n_planes;
  }
  if (steps > 8192) return Fail(HB_EINVAL, "%llu fold steps exceed 8192", (unsigned long long)steps);
  // the kernels address A and W words with 32-bit byte offsets from the
  // (moved) A base and from w
  const uint64_t quads = (d->m + 3) / 4, a_row = d->a_stride ? d->a_stride : d->kb_total;
  uint64_t a_end = 0;
  *mixed = false;
  for (uint32_t p = 0; p < d->n_pieces; ++p) {
    const hb_piece& pc = d->pieces[p];
    a_end = std::max(a_end, (quads - 1) * a_row + std::max<uint64_t>(pc.kb_offset, pc.a_word) + pc.kb);
    if (PieceShift(*d, p) != PieceShift(*d, 0)) *mixed = true;
  }
  const bool panels = (d->flags & HB_LINEAR_PANELS) != 0;
  const bool w8p = (d->flags & HB_LINEAR_W8_PANELS) != 0;
  const uint64_t w_bytes = w8p ? hb::W8PanelBytes(d->n, d->kb_total)
                           : panels ? hb::PanelBytes(d->n, d->kb_total)
                                    : (uint64_t)(d->n / 8) * d->kb_total * hb::kDdrWord;
  if (a_end * hb::kDdrWord > (1ull << 32) || w_bytes > (1ull << 32))
    return Fail(HB_EINVAL, "A or W spans more than 4 GiB");
  if (!d->a) return Fail(HB_EINVAL, "null A");
  // C may be left out (null) where the layer keeps only its requantized
  // words: the fp32 result then stays in the kernel, as in the NPU's FBUF
  if (!d->c && (!d->q_out || d->onto))
    return Fail(HB_EINVAL, "null C needs q_out and no onto");
  if (d->n_ops > HB_MAX_EP_OPS) return Fail(HB_EINVAL, "n_ops = %u", d->n_ops);
  if (d->q_out && d->n % 32 != 0) return Fail(HB_EINVAL, "quantized output needs n %% 32 == 0");
  if (reinterpret_cast<uintptr_t>(d->c) % 4 != 0 || reinterpret_cast<uintptr_t>(d->q_out) % 4 != 0)
    return Fail(HB_EINVAL, "C and q_out must be 4-byte aligned");
  const bool fp8 = (d->flags & HB_LINEAR_A_FP8) != 0;
  if (d->flags &
          ~(uint32_t)(HB_LINEAR_FAST | HB_LINEAR_PANELS | HB_LINEAR_W8_PANELS | HB_LINEAR_A_FP8) ||
      (panels && w8p))
    return Fail(HB_EINVAL, "flags = %u", d->flags);
  if (fp8 && (d->n_planes != 1 || d->modes[0] != 0 || w8p))
    return Fail(HB_EINVAL, "MXFP8 activations take one MXFP4 plane (modes {0})");
  for (uint32_t l = 0; panels && l < d->n_planes; ++l)
    if (reinterpret_cast<uintptr_t>(d->w[l]) % 16 != 0)
      return Fail(HB_EINVAL, "weight panels must be 16-byte aligned");
  if (w8p) {
    if (d->n_planes != 2 || d->modes[0] != 1 || d->modes[1] != 2 || d->w[1] != d->w[0])
      return Fail(HB_EINVAL, "W8 panels: planes {W8_HI, W8_LO} with w[0] == w[1]");
    if (reinterpret_cast<uintptr_t>(d->w[0]) % 16 != 0 ||
        reinterpret_cast<uintptr_t>(d->a) % 16 != 0)
      return Fail(HB_EINVAL, "W8 panels: A and the panels must be 16-byte aligned");
    if (d->n_pieces != 1 || d->pieces[0].kb_offset != 0 || d->pieces[0].kb != d->kb_total)
      return Fail(HB_EUNSUPPORTED, "W8 panels take one piece over every block");
  }
  std::memset(g, 0, sizeof *g);
  for (uint32_t o = 0; o < d->n_ops; ++o) {
    const hb_ep_op& op = d->ops[o];
    switch (op.op) {
      case HB_EP_ADDP:
      case HB_EP_MULP:
        if (!op.vec) return Fail(HB_EINVAL, "op %u needs a column vector", o);
        break;
      case HB_EP_ACT_MUL:
      case HB_EP_ADD:
        if (!op.x2) return Fail(HB_EINVAL, "op %u needs x2", o);
        [[fallthrough]];
      case HB_EP_ACT:
        if (op.op != HB_EP_ADD && !d->tbuf) return Fail(HB_EINVAL, "op %u needs TBUF", o);
        break;
      case HB_EP_SCALE:
      case HB_EP_COPY:
      case HB_EP_RELU:
        break;
      default: return Fail(HB_EUNSUPPORTED, "epilogue op %u is not supported", op.op);
    }
    g->op_kind[o] = op.op;
    g->op_imm[o] = op.imm;
    g->op_vec[o] = reinterpret_cast<const uint32_t*>(op.vec);
    g->op_x2[o] = reinterpret_cast<const uint32_t*>(op.x2);
  }
  g->n_ops = d->n_ops;
  g->a = static_cast<const uint8_t*>(d->a) + PieceShift(*d, 0) * (int64_t)hb::kDdrWord;
  g->w[0] = static_cast<const uint8_t*>(d->w[0]);
  g->w[1] = static_cast<const uint8_t*>(d->n_planes > 1 ? d->w[1] : d->w[0]);
  g->c = reinterpret_cast<uint32_t*>(d->c);
  g->quads = (d->m + 3) / 4;
  g->groups = d->n / 8;
  g->m = d->m;
  g->n = d->n;
  g->kb_total = d->kb_total;
  g->a_row = (uint32_t)a_row;
  g->n_pieces = d->n_pieces;
  for (uint32_t p = 0; p < d->n_pieces; ++p) {
    g->piece_off[p] = d->pieces[p].kb_offset;
    g->piece_kb[p] = d->pieces[p].kb;
  }
  g->n_planes = d->n_planes;
  g->modes[0] = d->modes[0];
  g->modes[1] = d->n_planes > 1 ? d->modes[1] : d->modes[0];
  g->total_steps = (uint32_t)steps;
  g->w_panels = panels ? 1u : 0u;
  g->w_fp6 = w8p ? 1u : 0u;
  g->a_fp8 = fp8 ? 1u : 0u;
  g->w_steps = (d->kb_total + 1) / 2;
  g->acc = d->onto ? 1u : 0u;
  g->tbuf = d->tbuf;
  g->q_out = static_cast<uint8_t*>(d->q_out);
  return HB_OK;
}

template <class T>
uint64_t Diff(const T* a, const T* b) {
  return (uint64_t)(reinterpret_cast<const uint8_t*>(b) - reinterpret_cast<const uint8_t*>(a));
}

int LinearChain(hb_ctx* ctx, const hb_linear_desc* d, uint32_t count, hb::FixedScratch* fixed);

// `fixed`: run without allocating, in that buffer (null: the context's
// workspace).
int LinearBatched(hb_ctx* ctx, const hb_linear_desc* d, uint32_t count,
                  hb::FixedScratch* fixed = nullptr) {
  if (!d || count < 1) return Fail(HB_EINVAL, "no layers");
  hb::GemmArgs g;
  bool mixed = false;
  if (int rc = LinearArgs(&d[0], &g, &mixed)) return rc;
  if (count > 1) {
    const hb_linear_desc& d0 = d[0];
    g.a_batch = Diff(d0.a, d[1].a);
    g.w_batch = Diff(d0.w[0], d[1].w[0]);
    g.c_batch = Diff(d0.c, d[1].c) / 4;
    g.q_batch = d0.q_out ? Diff(d0.q_out, d[1].q_out) : 0;
    for (uint32_t o = 0; o < d0.n_ops; ++o) {
      g.op_vec_batch[o] = d0.ops[o].vec ? Diff(d0.ops[o].vec, d[1].ops[o].vec) / 4 : 0;
      g.op_x2_batch[o] = d0.ops[o].x2 ? Diff(d0.ops[o].x2, d[1].ops[o].x2) / 4 : 0;
    }
    for (uint32_t i = 1; i < count; ++i) {
      const hb_linear_desc& x = d[i];
      bool same = x.m == d0.m && x.n == d0.n && x.kb_total == d0.kb_total &&
                  x.a_stride == d0.a_stride &&
                  x.n_planes == d0.n_planes && x.flags == d0.flags && x.onto == d0.onto &&
                  x.n_pieces == d0.n_pieces && x.n_ops == d0.n_ops && x.tbuf == d0.tbuf &&
                  (x.q_out != nullptr) == (d0.q_out != nullptr) &&
                  (x.c != nullptr) == (d0.c != nullptr) &&
                  Diff(d0.a, x.a) == i * g.a_batch && Diff(d0.w[0], x.w[0]) == i * g.w_batch &&
                  (x.n_planes < 2 || Diff(d0.w[1], x.w[1]) == i * g.w_batch) &&
                  Diff(d0.c, x.c) == i * g.c_batch * 4 &&
                  (!x.q_out || Diff(d0.q_out, x.q_out) == i * g.q_batch);
      for (uint32_t l = 0; same && l < d0.n_planes; ++l) same = x.modes[l] == d0.modes[l];
      for (uint32_t p = 0; same && p < d0.n_pieces; ++p)
        same = x.pieces[p].kb_offset == d0.pieces[p].kb_offset && x.pieces[p].kb == d0.pieces[p].kb &&
               (d0.a_stride == 0 || x.pieces[p].a_word == d0.pieces[p].a_word);
      for (uint32_t o = 0; same && o < d0.n_ops; ++o) {
        const hb_ep_op &a = d0.ops[o], &b = x.ops[o];
        same = a.op == b.op && a.imm == b.imm && (a.vec != nullptr) == (b.vec != nullptr) &&
               (a.x2 != nullptr) == (b.x2 != nullptr) &&
               (!a.vec || Diff(a.vec, b.vec) == i * g.op_vec_batch[o] * 4) &&
               (!a.x2 || Diff(a.x2, b.x2) == i * g.op_x2_batch[o] * 4);
      }
      if (!same) return Fail(HB_EINVAL, "layer %u differs in shape, schedule, ops or stride", i);
    }
    if (g.w_fp6 && (g.a_batch % 16 != 0 || g.w_batch % 16 != 0))
      return Fail(HB_EINVAL, "W8 panels: layers' A and panels must be 16-byte aligned");
  }
  if (mixed) {  // the runs of the chain meet in C
    if (!d[0].c) return Fail(HB_EINVAL, "pieces at different A offsets need C");
    return LinearChain(ctx, d, count, fixed);
  }
  hipError_t err = hb::LaunchLinear(g, count, (d[0].flags & HB_LINEAR_FAST) != 0, ctx->ws,
                                    ctx->stream, fixed);
  if (err == hipErrorOutOfMemory && fixed != nullptr && fixed->need > fixed->bytes)
    return Fail(HB_ENOMEM, "layer needs %zu bytes of K-split scratch; the no-allocation entry point holds %zu",
                fixed->need, fixed->bytes);
  if (err != hipSuccess) return HipFail(err, "linear launch");
  return HB_OK;
}

// A layer whose pieces' A words sit at different offsets from their W blocks
// runs as a chain of launches, one per run of consecutive pieces with one
// offset.  The fold is pieces-outer, so starting each run from the previous
// one's C folds in the same order; the ops and the requantize go with the
// last run.  The descriptors were validated as a whole.
int LinearChain(hb_ctx* ctx, const hb_linear_desc* d, uint32_t count, hb::FixedScratch* fixed) {
  std::vector<hb_linear_desc> part(d, d + count);
  for (uint32_t p0 = 0, p1; p0 < d[0].n_pieces; p0 = p1) {
    for (p1 = p0 + 1; p1 < d[0].n_pieces && PieceShift(d[0], p1) == PieceShift(d[0], p0);) ++p1;
    const bool last = p1 == d[0].n_pieces;
    for (uint32_t i = 0; i < count; ++i) {
      hb_linear_desc& x = part[i];
      x = d[i];
      x.n_pieces = p1 - p0;
      for (uint32_t p = p0; p < p1; ++p) x.pieces[p - p0] = d[i].pieces[p];
      x.onto = p0 > 0 ? 1u : d[i].onto;
      if (!last) {
        x.n_ops = 0;
        x.q_out = nullptr;
      }
    }
    if (int rc = LinearBatched(ctx, part.data(), count, fixed)) return rc;
  }
  return HB_OK;
}

}  // namespace

extern "C" {

int hb_abi_version(void) { return HB_ABI_VERSION; }

const char* hb_last_error(void) { return g_error.c_str(); }

int hb_ctx_create(int device, hb_ctx** out) {
  if (!out) return Fail(HB_EINVAL, "null output");
  int count = 0;
  HB_HIP(hipGetDeviceCount(&count));
  if (device < 0 || device >= count) return Fail(HB_EINVAL, "device %d of %d", device, count);
  HB_HIP(hipSetDevice(device));
  if (int rc = ScratchSetUp(device)) return rc;
  hb_ctx* ctx = new (std::nothrow) hb_ctx;
  if (!ctx) return Fail(HB_ENOMEM, "context");
  ctx->device = device;
  hipError_t err = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipMalloc(&ctx->d_flag, sizeof(uint32_t));
  // the workspace starts at the no-allocation path's size, so a layer whose
  // K splits fit in it never allocates after the context is created
  if (err == hipSuccess) err = hb::GrowWorkspace(ctx->ws, HB_NOALLOC_SCRATCH_BYTES, ctx->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
  if (err != hipSuccess) {
    hb::FreeWorkspace(ctx->ws);
    if (ctx->d_flag) (void)hipFree(ctx->d_flag);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return HipFail(err, "context create");
  }
  ctx->own_stream = true;
  *out = ctx;
  return HB_OK;
}

int hb_ctx_destroy(hb_ctx* ctx) {
  if (!ctx) return HB_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->d_flag) (void)hipFree(ctx->d_flag);
  hb::FreeWorkspace(ctx->ws);
  if (ctx->own_stream && ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return HB_OK;
}

int hb_ctx_set_stream(hb_ctx* ctx, void* hip_stream) {
  if (int rc = Enter(ctx)) return rc;
  if (ctx->own_stream && ctx->stream) {
    HB_HIP(hipStreamSynchronize(ctx->stream));
    HB_HIP(hipStreamDestroy(ctx->stream));
  }
  ctx->stream = static_cast<hipStream_t>(hip_stream);
  ctx->own_stream = false;
  return HB_OK;
}

int hb_ctx_synchronize(hb_ctx* ctx) {
  if (int rc = Enter(ctx)) return rc;
  HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

int hb_onchip_create(hb_ctx* ctx, hb_onchip** out) {
  if (int rc = Enter(ctx)) return rc;
  if (!out) return Fail(HB_EINVAL, "null output");
  hb_onchip* o = new (std::nothrow) hb_onchip;
  if (!o) return Fail(HB_ENOMEM, "onchip");
  o->ctx = ctx;
  hipError_t err = hipSuccess;
  const size_t sizes[5] = {(size_t)HB_ABUF_DEPTH * HB_ABUF_WORD_BYTES,
                           (size_t)HB_WBUF_DEPTH * HB_WBUF_WORD_BYTES,
                           (size_t)HB_FBUF_DEPTH * HB_FBUF_WORD_BYTES,
                           (size_t)HB_PBUF_DEPTH * HB_PBUF_WORD_BYTES,
                           (size_t)HB_TBUF_DEPTH * HB_TBUF_WORD_BYTES};
  void** ptrs[5] = {(void**)&o->abuf, (void**)&o->wbuf, (void**)&o->fbuf, (void**)&o->pbuf,
                    (void**)&o->tbuf};
  for (int i = 0; i < 5 && err == hipSuccess; ++i) {
    err = hipMalloc(ptrs[i], sizes[i]);
    if (err == hipSuccess) err = hipMemsetAsync(*ptrs[i], 0, sizes[i], ctx->stream);
  }
  if (err == hipSuccess) err = hipMalloc(&o->temp, (size_t)kVecTempWords * 128);
  if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
  if (err != hipSuccess) {
    hb_onchip_destroy(o);
    return HipFail(err, "onchip create");
  }
  *out = o;
  return HB_OK;
}

int hb_onchip_destroy(hb_onchip* o) {
  if (!o) return HB_OK;
  if (o->ctx) {
    (void)hipSetDevice(o->ctx->device);
    (void)hipStreamSynchronize(o->ctx->stream);
  }
  void* ptrs[6] = {o->abuf, o->wbuf, o->fbuf, o->pbuf, o->tbuf, o->temp};
  for (void* p : ptrs)
    if (p) (void)hipFree(p);
  delete o;
  return HB_OK;
}

static int Transfer(hb_onchip* o, int mem, uint32_t first, uint32_t count, void* host,
                    bool upload) {
  if (!o) return Fail(HB_EINVAL, "null onchip");
  if (int rc = Enter(o->ctx)) return rc;
  const MemInfo info = Info(mem);
  if (info.depth == 0) return Fail(HB_EINVAL, "memory id %d", mem);
  if ((uint64_t)first + count > info.depth)
    return Fail(HB_EINVAL, "words [%u, %u) outside depth %u", first, first + count, info.depth);
  if (count == 0) return HB_OK;
  if (!host) return Fail(HB_EINVAL, "null host buffer");
  uint8_t* dev = Image(o, mem) + (size_t)first * info.word;
  const size_t bytes = (size_t)count * info.word;
  if (upload)
    HB_HIP(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, o->ctx->stream));
  else
    HB_HIP(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, o->ctx->stream));
  HB_HIP(hipStreamSynchronize(o->ctx->stream));
  return HB_OK;
}

int hb_onchip_upload(hb_onchip* o, int mem, uint32_t first, uint32_t count, const void* host) {
  return Transfer(o, mem, first, count, const_cast<void*>(host), true);
}

int hb_onchip_download(hb_onchip* o, int mem, uint32_t first, uint32_t count, void* host) {
  return Transfer(o, mem, first, count, host, false);
}

int hb_onchip_device_ptr(hb_onchip* o, int mem, void** device) {
  if (!o || !device) return Fail(HB_EINVAL, "null argument");
  if (Info(mem).depth == 0) return Fail(HB_EINVAL, "memory id %d", mem);
  *device = Image(o, mem);
  return HB_OK;
}

int hb_gemm_decode(const uint8_t word[16], hb_gemm_cmd* out) {
  if (!word || !out) return Fail(HB_EINVAL, "null argument");
  const uint32_t opcode = Field(word, 120, 8);
  if (opcode != 4) return Fail(HB_EINVAL, "opcode %u is not GEMM (4)", opcode);
  // isa::gemm field map (include/hotarubi/isa.hpp:75-84)
  out->a_base = Field(word, 92, 20);
  out->a_stride = Field(word, 82, 10);
  out->kb = Field(word, 72, 10);
  out->m = Field(word, 62, 10);
  out->w_base = Field(word, 42, 20);
  out->w_stride = Field(word, 32, 10);
  out->n8 = Field(word, 24, 8);
  out->c_base = Field(word, 4, 20);
  out->wmode = Field(word, 2, 2);
  out->acc = Field(word, 1, 1);
  return HB_OK;
}

int hb_gemm_encode(const hb_gemm_cmd* c, uint8_t word[16]) {
  if (!c || !word) return Fail(HB_EINVAL, "null argument");
  std::memset(word, 0, 16);
  SetField(word, 120, 8, 4);
  SetField(word, 92, 20, c->a_base);
  SetField(word, 82, 10, c->a_stride);
  SetField(word, 72, 10, c->kb);
  SetField(word, 62, 10, c->m);
  SetField(word, 42, 20, c->w_base);
  SetField(word, 32, 10, c->w_stride);
  SetField(word, 24, 8, c->n8);
  SetField(word, 4, 20, c->c_base);
  SetField(word, 2, 2, c->wmode);
  SetField(word, 1, 1, c->acc ? 1u : 0u);
  return HB_OK;
}

int hb_gemm_check(const hb_gemm_cmd* cmd) {
  if (!cmd) return Fail(HB_EINVAL, "null command");
  return CheckGemm(cmd);
}

int hb_gemm_access(const hb_gemm_cmd* cmd, uint8_t* ra, uint8_t* rw, uint8_t* rf, uint8_t* wf) {
  if (!cmd) return Fail(HB_EINVAL, "null command");
  if (int rc = CheckGemm(cmd)) return rc;
  if (ra) std::memset(ra, 0, HB_ABUF_DEPTH);
  if (rw) std::memset(rw, 0, HB_WBUF_DEPTH);
  if (rf) std::memset(rf, 0, HB_FBUF_DEPTH);
  if (wf) std::memset(wf, 0, HB_FBUF_DEPTH);
  const uint32_t mask = hb::kAddrMask;
  for (uint32_t g = 0; g < cmd->n8; ++g) {
    if (rw)
      for (uint32_t b = 0; b < cmd->kb; ++b)
        rw[((cmd->w_base + g * cmd->w_stride + b) & mask) % HB_WBUF_DEPTH] = 1;
    for (uint32_t q = 0; q < cmd->m / 4; ++q) {
      const uint32_t c = ((cmd->c_base + q * cmd->n8 + g) & mask) % HB_FBUF_DEPTH;
      if (rf && cmd->acc) rf[c] = 1;
      if (ra)
        for (uint32_t b = 0; b < cmd->kb; ++b)
          ra[((cmd->a_base + q * cmd->a_stride + b) & mask) % HB_ABUF_DEPTH] = 1;
      if (wf) wf[c] = 1;
    }
  }
  return HB_OK;
}

int hb_gemm_exec(hb_ctx* ctx, const hb_gemm_cmd* cmd, hb_onchip* o) {
  return GemmExec(ctx, cmd, o, true);
}

int hb_gemm_exec_async(hb_ctx* ctx, const hb_gemm_cmd* cmd, hb_onchip* o) {
  return GemmExec(ctx, cmd, o, false);
}

uint64_t hb_gemm_cycles(const hb_gemm_cmd* c, uint32_t fixed_cycles) {
  if (!c) return 0;
  return (uint64_t)c->n8 * (c->m / 32) * c->kb * 8u + fixed_cycles;
}

int hb_vec_exec(hb_ctx* ctx, const hb_vec_cmd* cmd, hb_onchip* o) { return VecExec(ctx, cmd, o); }

int hb_rows(hb_ctx* ctx, const hb_rows_desc* d) { return Rows(ctx, d, true); }
int hb_rows_async(hb_ctx* ctx, const hb_rows_desc* d) { return Rows(ctx, d, false); }

int hb_linear_async(hb_ctx* ctx, const hb_linear_desc* d) {
  if (int rc = Enter(ctx)) return rc;
  return LinearBatched(ctx, d, 1);
}

int hb_linear(hb_ctx* ctx, const hb_linear_desc* d) {
  if (int rc = hb_linear_async(ctx, d)) return rc;
  HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

int hb_linear_batched_async(hb_ctx* ctx, const hb_linear_desc* d, uint32_t count) {
  if (int rc = Enter(ctx)) return rc;
  return LinearBatched(ctx, d, count);
}

int hb_linear_group_async(hb_ctx* ctx, const hb_linear_desc* d, uint32_t count) {
  if (int rc = Enter(ctx)) return rc;
  if (!d || count < 1 || count > HB_MAX_GROUP)
    return Fail(HB_EINVAL, "a group holds 1 to %d layers, not %u", HB_MAX_GROUP, count);
  hb::SplitGroup grp;
  std::memset(&grp, 0, sizeof grp);
  bool fuse = true;
  for (uint32_t i = 0; i < count; ++i) {
    bool mixed = false;
    if (int rc = LinearArgs(&d[i], &grp.g[i], &mixed)) return rc;
    const hb::GemmArgs& g = grp.g[i];
    fuse = fuse && !mixed && (d[i].flags & HB_LINEAR_FAST) && !g.w_fp6 && !g.a_fp8 &&
           hb::FastEligible(g) &&
           hb::SplitEligible(g, 1) && g.n_planes == grp.g[0].n_planes &&
           (g.n_pieces > 1) == (grp.g[0].n_pieces > 1);
  }
  // Fused pairs: a later layer whose ACT_MUL reads an earlier one's C over
  // the same m x n folds beside it in its workgroups and reads its values
  // there.
  constexpr uint32_t kNone = hb::kMaxGroup;
  uint32_t partner[hb::kMaxGroup], pair_op[hb::kMaxGroup];
  bool second[hb::kMaxGroup] = {};
  for (uint32_t i = 0; i < count; ++i) partner[i] = kNone;
  for (uint32_t j = 1; j < count && fuse; ++j)
    for (uint32_t o = 0; o < d[j].n_ops && !second[j]; ++o) {
      if (d[j].ops[o].op != HB_EP_ACT_MUL) continue;
      for (uint32_t i = 0; i < j; ++i)
        if (partner[i] == kNone && !second[i] && d[j].ops[o].x2 == d[i].c && d[i].m == d[j].m &&
            d[i].n == d[j].n) {
          partner[i] = j;
          pair_op[i] = o;
          second[j] = true;
          break;
        }
    }
  // Every ACT_MUL over an earlier layer's C must have become that layer's
  // pair: a second consumer of one producer, or a consumer of a pair's
  // second layer, would read C while the producer's workgroups still write
  // it in the shared launch.  Such a group runs one layer at a time.
  for (uint32_t j = 1; j < count && fuse; ++j)
    for (uint32_t o = 0; o < d[j].n_ops && fuse; ++o) {
      if (d[j].ops[o].op != HB_EP_ACT_MUL) continue;
      for (uint32_t i = 0; i < j && fuse; ++i)
        if (d[j].ops[o].x2 == d[i].c && !(partner[i] == j && pair_op[i] == o)) fuse = false;
    }
  if (!fuse) {  // one launch per layer, in order
    for (uint32_t i = 0; i < count; ++i)
      if (int rc = LinearBatched(ctx, &d[i], 1)) return rc;
    return HB_OK;
  }
  // Split plans: a lone layer's as its own launch would take (at most
  // kMaxSplitWaves splits), a pair's layers at most half that each (they
  // share a workgroup).  Where the grid would not fit the CUs in one round,
  // the caps halve (pairs first): a second round costs more than longer K
  // ranges per wave.
  uint32_t cap1 = hb::kMaxSplitWaves, cap2 = hb::kMaxSplitWaves / 2, waves = 1, end = 0;
  const uint64_t cus = (uint64_t)hb::DeviceCus();
  for (;;) {
    waves = hb::kSplitFinishWaves;
    end = 0;
    for (uint32_t i = 0; i < count; ++i) {
      if (second[i]) continue;
      hb::SplitPlan(grp.g[i], partner[i] == kNone ? cap1 : cap2);
      uint32_t w = grp.g[i].splits;
      if (partner[i] != kNone) {
        hb::SplitPlan(grp.g[partner[i]], cap2);
        w += grp.g[partner[i]].splits;
      }
      waves = std::max(waves, w);
      end += grp.g[i].gx * grp.g[i].gy;
    }
    const uint64_t resident = cus * std::max(1u, hb::kSplitWavesPerCu / waves);
    if (end <= resident || (cap1 == 1 && cap2 == 1)) break;
    if (cap2 > 1) cap2 /= 2;
    else cap1 /= 2;
  }
  end = 0;
  for (uint32_t i = 0; i < count; ++i) {
    grp.g[i].fast_ep = 1u;
    if (second[i]) continue;
    const uint32_t u = grp.units++;
    end += grp.g[i].gx * grp.g[i].gy;
    grp.tile_end[u] = end;
    grp.first[u] = i;
    grp.second[u] = partner[i];
    grp.x2_op[u] = partner[i] == kNone ? 0u : pair_op[i];
  }
  const hipError_t err = hb::LaunchSplitGroup(grp, waves, ctx->stream);
  if (err != hipSuccess) return HipFail(err, "group launch");
  return HB_OK;
}

int hb_linear_noalloc_async(hb_ctx* ctx, const hb_linear_desc* d, uint32_t count) {
  if (int rc = Enter(ctx)) return rc;
  void* p = nullptr;
  {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (ctx->device >= 0 && ctx->device < kMaxDevices) p = g_scratch_ptr[ctx->device];
  }
  if (p == nullptr) return Fail(HB_EDEVICE, "no scratch on device %d", ctx->device);
  hb::FixedScratch fixed{p, HB_NOALLOC_SCRATCH_BYTES, 0};
  return LinearBatched(ctx, d, count, &fixed);
}

uint64_t hb_panel_bytes(uint32_t n, uint32_t kb_total) {
  if (n < 8 || n % 8 != 0 || kb_total < 1) return 0;
  return hb::PanelBytes(n, kb_total);
}

namespace {
int PanelConvert(hb_ctx* ctx, const void* src, uint32_t n, uint32_t kb_total, void* dst,
                 bool pack) {
  if (int rc = Enter(ctx)) return rc;
  if (!src || !dst) return Fail(HB_EINVAL, "null weights");
  if (n < 8 || n % 8 != 0 || kb_total < 1)
    return Fail(HB_EINVAL, "weights n = %u, kb_total = %u: need n %% 8 == 0, kb_total >= 1", n,
                kb_total);
  if (reinterpret_cast<uintptr_t>(src) % 16 != 0 || reinterpret_cast<uintptr_t>(dst) % 16 != 0)
    return Fail(HB_EINVAL, "weights must be 16-byte aligned");
  const uint8_t* s = static_cast<const uint8_t*>(src);
  uint8_t* d = static_cast<uint8_t*>(dst);
  const hipError_t err = pack ? hb::LaunchPackPanels(s, n, kb_total, d, ctx->stream)
                              : hb::LaunchUnpackPanels(s, n, kb_total, d, ctx->stream);
  if (err != hipSuccess) return HipFail(err, pack ? "pack launch" : "unpack launch");
  HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}
}  // namespace

int hb_pack_weights(hb_ctx* ctx, const void* w, uint32_t n, uint32_t kb_total, void* panels) {
  return PanelConvert(ctx, w, n, kb_total, panels, true);
}

int hb_unpack_weights(hb_ctx* ctx, const void* panels, uint32_t n, uint32_t kb_total, void* w) {
  return PanelConvert(ctx, panels, n, kb_total, w, false);
}

uint64_t hb_w8_panel_bytes(uint32_t n, uint32_t kb_total) {
  if (n < 8 || n % 8 != 0 || kb_total < 1) return 0;
  return hb::W8PanelBytes(n, kb_total);
}

namespace {
int W8Convert(hb_ctx* ctx, const void* hi, const void* lo, uint32_t n, uint32_t kb_total,
              const void* in_panels, void* out_panels, void* out_hi, void* out_lo) {
  if (int rc = Enter(ctx)) return rc;
  const bool pack = out_panels != nullptr;
  const void* bufs[3] = {pack ? hi : in_panels, pack ? lo : out_hi, pack ? out_panels : out_lo};
  for (const void* b : bufs) {
    if (!b) return Fail(HB_EINVAL, "null weights");
    if (reinterpret_cast<uintptr_t>(b) % 16 != 0)
      return Fail(HB_EINVAL, "weights must be 16-byte aligned");
  }
  if (n < 8 || n % 8 != 0 || kb_total < 1)
    return Fail(HB_EINVAL, "weights n = %u, kb_total = %u: need n %% 8 == 0, kb_total >= 1", n,
                kb_total);
  if (hb::W8PanelBytes(n, kb_total) > (1ull << 32))
    return Fail(HB_EINVAL, "W8 panels of more than 4 GiB");
  const hipError_t err =
      pack ? hb::LaunchPackW8(static_cast<const uint8_t*>(hi), static_cast<const uint8_t*>(lo),
                              n, kb_total, static_cast<uint8_t*>(out_panels), ctx->stream)
           : hb::LaunchUnpackW8(static_cast<const uint8_t*>(in_panels), n, kb_total,
                                static_cast<uint8_t*>(out_hi), static_cast<uint8_t*>(out_lo),
                                ctx->stream);
  if (err != hipSuccess) return HipFail(err, pack ? "W8 pack launch" : "W8 unpack launch");
  HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}
}  // namespace

int hb_pack_w8(hb_ctx* ctx, const void* w_hi, const void* w_lo, uint32_t n, uint32_t kb_total,
               void* panels) {
  return W8Convert(ctx, w_hi, w_lo, n, kb_total, nullptr, panels, nullptr, nullptr);
}

int hb_unpack_w8(hb_ctx* ctx, const void* panels, uint32_t n, uint32_t kb_total, void* w_hi,
                 void* w_lo) {
  if (!panels) return Fail(HB_EINVAL, "null weights");
  return W8Convert(ctx, nullptr, nullptr, n, kb_total, panels, nullptr, w_hi, w_lo);
}

}  // extern "C"

namespace {

int EncodeMx(hb_ctx* ctx, const float* x, uint32_t rows, uint32_t cols, void* out, bool fp8) {
  if (int rc = Enter(ctx)) return rc;
  if (!x || !out || rows < 1 || cols < 1) return Fail(HB_EINVAL, "bad encode arguments");
  HB_HIP(hipMemsetAsync(ctx->d_flag, 0, sizeof(uint32_t), ctx->stream));
  hipError_t err = hb::LaunchEncodeMxint8(x, rows, cols, static_cast<uint8_t*>(out),
                                          ctx->d_flag, ctx->stream, fp8);
  if (err != hipSuccess) return HipFail(err, "encode launch");
  uint32_t flag = 0;
  HB_HIP(hipMemcpyAsync(&flag, ctx->d_flag, sizeof flag, hipMemcpyDeviceToHost, ctx->stream));
  HB_HIP(hipStreamSynchronize(ctx->stream));
  if (flag) return Fail(HB_EINVAL, "%s input is infinite or NaN", fp8 ? "MXFP8" : "MXINT8");
  return HB_OK;
}

}  // namespace

extern "C" {

int hb_encode_mxint8(hb_ctx* ctx, const float* x, uint32_t rows, uint32_t cols, void* out) {
  return EncodeMx(ctx, x, rows, cols, out, false);
}

int hb_encode_mxfp8(hb_ctx* ctx, const float* x, uint32_t rows, uint32_t cols, void* out) {
  return EncodeMx(ctx, x, rows, cols, out, true);
}

}  // extern "C"

namespace {
// Runs one preparation launch with the context's flag word cleared first;
// nonzero flag: the reference's rejection, as HB_EINVAL with `what`.
template <typename Launch>
int Prepare(hb_ctx* ctx, Launch launch, const char* name, const char* what) {
  HB_HIP(hipMemsetAsync(ctx->d_flag, 0, sizeof(uint32_t), ctx->stream));
  const hipError_t err = launch(ctx->d_flag);
  if (err != hipSuccess) return HipFail(err, name);
  uint32_t flag = 0;
  HB_HIP(hipMemcpyAsync(&flag, ctx->d_flag, sizeof flag, hipMemcpyDeviceToHost, ctx->stream));
  HB_HIP(hipStreamSynchronize(ctx->stream));
  if (flag) return Fail(HB_EINVAL, "%s", what);
  return HB_OK;
}
}  // namespace

extern "C" {

int hb_w8_from_fp32(hb_ctx* ctx, const float* w, uint32_t rows, uint32_t cols,
                    uint32_t out_rows, void* w_hi, void* w_lo) {
  if (int rc = Enter(ctx)) return rc;
  if (!w || !w_hi || !w_lo) return Fail(HB_EINVAL, "null weights");
  if (rows < 1 || cols < 1 || out_rows < rows || out_rows % 8 != 0)
    return Fail(HB_EINVAL, "cannot pad %u rows to %u (a multiple of 8 at least rows)", rows,
                out_rows);
  if (reinterpret_cast<uintptr_t>(w_hi) % 16 != 0 || reinterpret_cast<uintptr_t>(w_lo) % 16 != 0)
    return Fail(HB_EINVAL, "weight words must be 16-byte aligned");
  return Prepare(ctx, [&](uint32_t* flag) {
    return hb::LaunchW8FromFp32(w, rows, cols, out_rows, static_cast<uint8_t*>(w_hi),
                                static_cast<uint8_t*>(w_lo), flag, ctx->stream);
  }, "W8 weight launch", "MXINT8 input is infinite or NaN");
}

int hb_mxfp4_canonical(hb_ctx* ctx, const uint8_t* codes, const uint8_t* scales, uint32_t rows,
                       uint32_t cols, int32_t exponent_shift, uint32_t out_rows, void* w) {
  if (int rc = Enter(ctx)) return rc;
  if (!codes || !scales || !w) return Fail(HB_EINVAL, "null weights");
  if (rows < 1 || cols < 32 || cols % 32 != 0 || out_rows < rows || out_rows % 8 != 0)
    return Fail(HB_EINVAL, "cannot pad a %ux%u MXFP4 matrix to %u rows", rows, cols, out_rows);
  if (reinterpret_cast<uintptr_t>(w) % 16 != 0)
    return Fail(HB_EINVAL, "weight words must be 16-byte aligned");
  return Prepare(ctx, [&](uint32_t* flag) {
    return hb::LaunchMxfp4Canonical(codes, scales, rows, cols, exponent_shift, out_rows,
                                    static_cast<uint8_t*>(w), flag, ctx->stream);
  }, "MXFP4 weight launch", "a canonical MXFP4 block exponent is outside E8M0");
}

}  // extern "C"

namespace {

int DmaSplit(hb_ctx* ctx, const void* src, uint64_t stride, uint32_t rows, uint32_t row_words,
             void* hi, void* lo, bool t32, bool sync) {
  if (int rc = Enter(ctx)) return rc;
  if (!src || !hi || !lo || rows < 1 || row_words < 1)
    return Fail(HB_EINVAL, "bad %s arguments", t32 ? "T32_SPLIT8" : "SPLIT8");
  if (stride % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(hi) % 16 != 0 || reinterpret_cast<uintptr_t>(lo) % 16 != 0)
    return Fail(HB_EINVAL, "%s buffers must be 16-byte aligned with a stride of whole 16-byte beats",
                t32 ? "T32_SPLIT8" : "SPLIT8");
  if (stride < (uint64_t)row_words * hb::kDdrWord)
    return Fail(HB_EINVAL, "%s row stride %llu is shorter than %u words",
                t32 ? "T32_SPLIT8" : "SPLIT8", (unsigned long long)stride, row_words);
  // the reference's Require texts (dma_engine.cpp:305-306, 380-382)
  if (!t32 && rows % 2 != 0) return Fail(HB_EBADCMD, "SPLIT8 with an odd number of rows %u", rows);
  if (t32 && rows % 8 != 0)
    return Fail(HB_EBADCMD, "T32_SPLIT8 with %u rows, not a multiple of 8", rows);
  const uint8_t* s = static_cast<const uint8_t*>(src);
  uint8_t* h = static_cast<uint8_t*>(hi);
  uint8_t* l = static_cast<uint8_t*>(lo);
  const hipError_t err = t32 ? hb::LaunchT32Split8(s, stride, rows, row_words, h, l, ctx->stream)
                             : hb::LaunchSplit8(s, stride, rows, row_words, h, l, ctx->stream);
  if (err != hipSuccess) return HipFail(err, t32 ? "T32_SPLIT8 launch" : "SPLIT8 launch");
  if (sync) HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

// Row format (dma_engine.cpp:96-125): the reference's checks in its order,
// then this backend's alignment needs.
int RowFormatCheck(uint32_t rows, uint32_t row_words, uint32_t tok, bool indexed,
                   uint32_t* token_bytes) {
  if (rows == 0 || row_words == 0)
    return Fail(HB_EBADCMD, "a DMA transfer with %u rows of %u words", rows, row_words);
  if (tok < 1 || tok > 32) return Fail(HB_EBADCMD, "row format with tok = %u", tok);
  const uint32_t bytes = (2 * tok + (tok > 16 ? 2u : 1u)) * 16u;
  const uint64_t units = (uint64_t)rows * row_words;
  if (units % 4 != 0)
    return Fail(HB_EBADCMD, "row format with %llu tokens, not a multiple of 4",
                (unsigned long long)units);
  if (!indexed && (uint64_t)row_words * (bytes / 16) >= 65536)
    return Fail(HB_EBADCMD, "row format with %u tokens of %u bytes per row", row_words, bytes);
  if (units * tok >= (1ull << 32)) return Fail(HB_EINVAL, "too many tokens");
  *token_bytes = bytes;
  return HB_OK;
}

bool Aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

int RowLoad(hb_ctx* ctx, const void* src, uint64_t stride, uint32_t rows, uint32_t row_words,
            uint32_t tok, const uint32_t* index, void* out, bool sync) {
  if (int rc = Enter(ctx)) return rc;
  if (!src || !out) return Fail(HB_EINVAL, "null row format buffer");
  uint32_t bytes = 0;
  if (int rc = RowFormatCheck(rows, row_words, tok, index != nullptr, &bytes)) return rc;
  if (!Aligned16(src) || !Aligned16(out) || (!index && stride % 16 != 0))
    return Fail(HB_EINVAL, "row format buffers must be 16-byte aligned, the stride whole beats");
  if (!index && stride < (uint64_t)row_words * bytes)
    return Fail(HB_EINVAL, "row stride %llu is shorter than %u tokens of %u bytes",
                (unsigned long long)stride, row_words, bytes);
  const hipError_t err = hb::LaunchRowLoad(static_cast<const uint8_t*>(src), stride, rows,
                                           row_words, tok, bytes, index,
                                           static_cast<uint8_t*>(out), ctx->stream);
  if (err != hipSuccess) return HipFail(err, "row format load launch");
  if (sync) HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

int RowStore(hb_ctx* ctx, const void* words, uint32_t rows, uint32_t row_words, uint32_t tok,
             void* dst, uint64_t stride, bool sync) {
  if (int rc = Enter(ctx)) return rc;
  if (!words || !dst) return Fail(HB_EINVAL, "null row format buffer");
  uint32_t bytes = 0;
  if (int rc = RowFormatCheck(rows, row_words, tok, false, &bytes)) return rc;
  if (!Aligned16(words) || !Aligned16(dst) || stride % 16 != 0)
    return Fail(HB_EINVAL, "row format buffers must be 16-byte aligned, the stride whole beats");
  if (stride < (uint64_t)row_words * bytes)
    return Fail(HB_EINVAL, "row stride %llu is shorter than %u tokens of %u bytes",
                (unsigned long long)stride, row_words, bytes);
  const hipError_t err = hb::LaunchRowStore(static_cast<const uint8_t*>(words), rows, row_words,
                                            tok, bytes, static_cast<uint8_t*>(dst), stride,
                                            ctx->stream);
  if (err != hipSuccess) return HipFail(err, "row format store launch");
  if (sync) HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

int Gacc(hb_ctx* ctx, const hb_gacc_desc* d, bool sync) {
  if (int rc = Enter(ctx)) return rc;
  if (!d || !d->base || !d->list || !d->out) return Fail(HB_EINVAL, "null GACC argument");
  // the reference's checks in its order (dma_engine.cpp Execute, Gather)
  if (d->slots == 0 || d->blocks == 0)
    return Fail(HB_EBADCMD, "a DMA transfer with %u rows of %u words", d->slots, d->blocks);
  if (d->blocks > 8) return Fail(HB_EBADCMD, "GACC with %u blocks per token", d->blocks);
  if (d->slots > 2047) return Fail(HB_EBADCMD, "GACC with %u slots", d->slots);
  if (d->quads < 1) return Fail(HB_EINVAL, "GACC over no quads");
  if (reinterpret_cast<uintptr_t>(d->list) % 16 != 0 || d->list_stride % 16 != 0 ||
      reinterpret_cast<uintptr_t>(d->base) % 16 != 0 || reinterpret_cast<uintptr_t>(d->out) % 16 != 0)
    return Fail(HB_EINVAL, "GACC lists, base and out must be 16-byte aligned");
  if (d->quads > 1 && d->list_stride < 16 + 128ull * d->slots)
    return Fail(HB_EINVAL, "GACC list stride %llu is shorter than a list of %u slots",
                (unsigned long long)d->list_stride, d->slots);
  hb::GaccArgs a{};
  a.base = static_cast<const uint8_t*>(d->base);
  a.list = static_cast<const uint8_t*>(d->list);
  a.list_stride = d->list_stride;
  a.quads = d->quads;
  a.slots = d->slots;
  a.blocks = d->blocks;
  a.w_stride = d->w_stride;
  a.accumulate = d->accumulate ? 1u : 0u;
  a.out = d->out;
  const hipError_t err = hb::LaunchGacc(a, ctx->stream);
  if (err != hipSuccess) return HipFail(err, "GACC launch");
  if (sync) HB_HIP(hipStreamSynchronize(ctx->stream));
  return HB_OK;
}

}  // namespace

extern "C" {

int hb_gacc(hb_ctx* ctx, const hb_gacc_desc* d) { return Gacc(ctx, d, true); }
int hb_gacc_async(hb_ctx* ctx, const hb_gacc_desc* d) { return Gacc(ctx, d, false); }

int hb_row_load(hb_ctx* ctx, const void* src, uint64_t row_stride, uint32_t rows,
                uint32_t row_words, uint32_t tok, const uint32_t* index, void* out) {
  return RowLoad(ctx, src, row_stride, rows, row_words, tok, index, out, true);
}
int hb_row_load_async(hb_ctx* ctx, const void* src, uint64_t row_stride, uint32_t rows,
                      uint32_t row_words, uint32_t tok, const uint32_t* index, void* out) {
  return RowLoad(ctx, src, row_stride, rows, row_words, tok, index, out, false);
}
int hb_row_store(hb_ctx* ctx, const void* words, uint32_t rows, uint32_t row_words, uint32_t tok,
                 void* dst, uint64_t row_stride) {
  return RowStore(ctx, words, rows, row_words, tok, dst, row_stride, true);
}
int hb_row_store_async(hb_ctx* ctx, const void* words, uint32_t rows, uint32_t row_words,
                       uint32_t tok, void* dst, uint64_t row_stride) {
  return RowStore(ctx, words, rows, row_words, tok, dst, row_stride, false);
}

int hb_split8(hb_ctx* ctx, const void* src, uint64_t src_stride, uint32_t rows, uint32_t row_words,
              void* hi, void* lo) {
  return DmaSplit(ctx, src, src_stride, rows, row_words, hi, lo, false, true);
}

int hb_split8_async(hb_ctx* ctx, const void* src, uint64_t src_stride, uint32_t rows,
                    uint32_t row_words, void* hi, void* lo) {
  return DmaSplit(ctx, src, src_stride, rows, row_words, hi, lo, false, false);
}

int hb_t32_split8(hb_ctx* ctx, const void* src, uint64_t src_stride, uint32_t rows,
                  uint32_t row_words, void* hi, void* lo) {
  return DmaSplit(ctx, src, src_stride, rows, row_words, hi, lo, true, true);
}

int hb_t32_split8_async(hb_ctx* ctx, const void* src, uint64_t src_stride, uint32_t rows,
                        uint32_t row_words, void* hi, void* lo) {
  return DmaSplit(ctx, src, src_stride, rows, row_words, hi, lo, true, false);
}

}  // extern "C"

// ---------------------------------------------------------- DDR images --

extern "C" {

int hb_image_create(hb_ctx* ctx, uint64_t capacity, hb_image** out) {
  if (!out) return Fail(HB_EINVAL, "null image");
  *out = nullptr;
  auto* img = new (std::nothrow) hb_image;
  if (!img) return Fail(HB_ENOMEM, "image bookkeeping");
  img->capacity = capacity;
  if (ctx != nullptr) {
    if (int rc = Enter(ctx)) {
      delete img;
      return rc;
    }
    img->ctx = ctx;
    if (capacity > 0) {
      const hipError_t err = hipMalloc(&img->bytes, capacity);
      if (err != hipSuccess) {
        delete img;
        return Fail(HB_ENOMEM, "image of %llu bytes: %s", (unsigned long long)capacity,
                    hipGetErrorString(err));
      }
      const hipError_t zero = hipMemset(img->bytes, 0, capacity);
      if (zero != hipSuccess) {
        (void)hipFree(img->bytes);
        delete img;
        return HipFail(zero, "image clear");
      }
    }
  }
  *out = img;
  return HB_OK;
}

void hb_image_destroy(hb_image* img) {
  if (!img) return;
  if (img->bytes) {
    (void)hipSetDevice(img->ctx->device);
    (void)hipFree(img->bytes);
  }
  delete img;
}

int hb_image_alloc(hb_image* img, const char* name, uint64_t size, uint64_t align,
                   uint64_t* offset) {
  if (!img || !name) return Fail(HB_EINVAL, "null image or name");
  if (align == 0) align = 4096;
  const auto found = img->index.find(name);
  if (img->reuse && found != img->index.end()) {
    const auto& region = img->regions[found->second].second;
    if (size > region.second)
      return Fail(HB_EINVAL, "region %s reused with %llu bytes but holds %llu", name,
                  (unsigned long long)size, (unsigned long long)region.second);
    if (offset) *offset = region.first;
    return HB_OK;
  }
  const uint64_t at = (img->end + align - 1) / align * align;
  if (at < img->end || at + size < at || at + size > img->capacity)
    return Fail(HB_EINVAL, "region %s of %llu bytes at %#llx exceeds the image of %llu bytes",
                name, (unsigned long long)size, (unsigned long long)at,
                (unsigned long long)img->capacity);
  if (found != img->index.end()) {
    img->regions[found->second].second = {at, size};
  } else {
    img->index.emplace(name, img->regions.size());
    img->regions.emplace_back(name, std::make_pair(at, size));
  }
  img->end = at + size;
  if (offset) *offset = at;
  return HB_OK;
}

void hb_image_set_reuse(hb_image* img, int reuse) {
  if (img) img->reuse = reuse != 0;
}

int hb_image_define(hb_image* img, const char* name, uint64_t offset, uint64_t size) {
  if (!img || !name) return Fail(HB_EINVAL, "null image or name");
  if (offset + size < offset || offset + size > img->end || img->index.count(name))
    return Fail(HB_EINVAL, "cannot define region %s at %#llx", name, (unsigned long long)offset);
  img->index.emplace(name, img->regions.size());
  img->regions.emplace_back(name, std::make_pair(offset, size));
  return HB_OK;
}

int hb_image_put(hb_image* img, uint64_t offset, const void* bytes, uint64_t size) {
  if (!img || (!bytes && size)) return Fail(HB_EINVAL, "null image or bytes");
  if (offset + size < offset || offset + size > img->capacity)
    return Fail(HB_EINVAL, "%llu bytes at %#llx exceed the image", (unsigned long long)size,
                (unsigned long long)offset);
  if (!img->bytes) return Fail(HB_EINVAL, "the image has no device memory");
  if (int rc = Enter(img->ctx)) return rc;
  if (size == 0) return HB_OK;
  HB_HIP(hipMemcpyAsync(img->bytes + offset, bytes, size, hipMemcpyHostToDevice,
                        img->ctx->stream));
  HB_HIP(hipStreamSynchronize(img->ctx->stream));
  return HB_OK;
}

int hb_image_get(const hb_image* img, uint64_t offset, void* bytes, uint64_t size) {
  if (!img || (!bytes && size)) return Fail(HB_EINVAL, "null image or bytes");
  if (offset + size < offset || offset + size > img->capacity)
    return Fail(HB_EINVAL, "%llu bytes at %#llx exceed the image", (unsigned long long)size,
                (unsigned long long)offset);
  if (!img->bytes) return Fail(HB_EINVAL, "the image has no device memory");
  if (int rc = Enter(img->ctx)) return rc;
  if (size == 0) return HB_OK;
  HB_HIP(hipMemcpyAsync(bytes, img->bytes + offset, size, hipMemcpyDeviceToHost,
                        img->ctx->stream));
  HB_HIP(hipStreamSynchronize(img->ctx->stream));
  return HB_OK;
}

int hb_image_region(const hb_image* img, const char* name, uint64_t* offset, uint64_t* size) {
  if (!img || !name) return Fail(HB_EINVAL, "null image or name");
  const auto found = img->index.find(name);
  if (found == img->index.end()) return Fail(HB_EINVAL, "no region named %s", name);
  const auto& region = img->regions[found->second].second;
  if (offset) *offset = region.first;
  if (size) *size = region.second;
  return HB_OK;
}

uint32_t hb_image_region_count(const hb_image* img) {
  return img ? (uint32_t)img->regions.size() : 0u;
}

int hb_image_region_at(const hb_image* img, uint32_t index, const char** name, uint64_t* offset,
                       uint64_t* size) {
  if (!img || index >= img->regions.size()) return Fail(HB_EINVAL, "no region %u", index);
  const auto& entry = img->regions[index];
  if (name) *name = entry.first.c_str();
  if (offset) *offset = entry.second.first;
  if (size) *size = entry.second.second;
  return HB_OK;
}

uint64_t hb_image_end(const hb_image* img) { return img ? img->end : 0u; }

void* hb_image_base(const hb_image* img) { return img ? img->bytes : nullptr; }

}  // extern "C"
