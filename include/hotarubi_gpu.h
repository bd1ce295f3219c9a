/*
 * hotarubi_gpu.h -- C ABI of the MI355X (gfx950) backend for hotarubi's
 * quantized GEMM instruction and its VEC epilogue.
 *
 * Three levels, all plain C (no torch or HIP types in the signatures):
 *
 *  1. Instruction level -- drop-in for the ISS GEMM and VEC engines.
 *     hb_gemm_exec replaces
 *        void iss::ExecuteGemm(const GemmCommand&, Memories&)
 *        (tools/iss/gemm_array.hpp:33, gemm_array.cpp:112-149)
 *     hb_vec_exec replaces, for library entries 0-9,
 *        void iss::VecEngine::Execute(const VecCommand&, Memories&)
 *        (tools/iss/vec_engine.hpp:87, vec_engine.cpp:163-209)
 *     on device-resident copies of the on-chip memories (hb_onchip) in the
 *     ISS's own word layout (tools/iss/memories.hpp:16-39): ABUF 8192 x 132 B,
 *     WBUF 2048 x 144 B, FBUF 4096 x 32 u32, PBUF 512 x 32 u32, TBUF 1024 u64.
 *
 *  2. Linear level -- the performance path.  hb_linear computes what the
 *     GEMM instruction sequence emitted by LinearEmitter::Emit
 *     (tools/compiler/kernels.cpp:343-395) computes, over the DDR word
 *     formats of PackAbuf (tools/runtime/formats.cpp:114-136) and PackWbuf
 *     (tools/compiler/tensors.cpp:66-90), followed by fused VEC epilogue ops
 *     (tools/compiler/vec_rom.cpp:314-349, tools/iss/lane.cpp:305-424) and an
 *     optional MXINT8 requantize (VecEngine::Store, vec_engine.cpp:447-458).
 *
 *  3. Formats -- hb_encode_mxint8 replaces EncodeMxint8 + PackAbuf
 *     (tools/runtime/formats.cpp:138-162, :114-136) for activations that
 *     are already in device memory.
 *
 * Arithmetic contract.  HB_EXACT (the default) is bitwise equal to the
 * reference for every input: exact per-block integer sums, exact block
 * values s*2^(ea+ew+SBIAS), an FP32 fold in block order with RNE, flush of
 * subnormals to +0, -0 -> +0, overflow to +-inf (tools/iss/fp32.hpp).
 * HB_FAST keeps the per-block products exact but lets the matrix cores
 * accumulate in their own order; it is only tolerance-equal (the measured
 * bound at hb_linear_desc.flags).
 *
 * Errors.  Every entry point returns HB_OK (0) or an hb_status code and
 * never aborts.  hb_last_error() gives the message of the calling thread's
 * last failure; for a rejected GEMM or VEC command it contains the same text
 * the reference passes to Fail (tools/runtime/require.cpp:10-13), e.g.
 * "GEMM m = 16 is not a multiple of 32 from 32 to 992".  A rejected command
 * leaves every image untouched.
 *
 * Threading.  One hb_ctx per host thread; a context is not re-entrant.
 * Calls are synchronous (results visible on return) unless the name ends in
 * _async, in which case they are ordered on the context's stream.
 */
#ifndef HOTARUBI_GPU_H_
#define HOTARUBI_GPU_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HB_ABI_VERSION 3

typedef enum hb_status {
  HB_OK = 0,
  HB_EBADCMD = 1,      /* a command the reference rejects with Fail */
  HB_EINVAL = 2,       /* bad argument to this API */
  HB_EUNSUPPORTED = 3, /* VEC entry outside 0-9, or mode not built */
  HB_EDEVICE = 4,      /* HIP runtime error */
  HB_ENOMEM = 5
} hb_status;

/* On-chip memory ids, the values of isa::Mem (include/hotarubi/isa.hpp:34-41). */
typedef enum hb_mem {
  HB_MEM_ABUF = 0,
  HB_MEM_WBUF = 1,
  HB_MEM_FBUF = 2,
  HB_MEM_PBUF = 3,
  HB_MEM_TBUF = 4
} hb_mem;

enum {
  HB_ABUF_DEPTH = 8192, HB_ABUF_WORD_BYTES = 132,
  HB_WBUF_DEPTH = 2048, HB_WBUF_WORD_BYTES = 144,
  HB_FBUF_DEPTH = 4096, HB_FBUF_WORD_BYTES = 128,
  HB_PBUF_DEPTH = 512,  HB_PBUF_WORD_BYTES = 128,
  HB_TBUF_DEPTH = 1024, HB_TBUF_WORD_BYTES = 8,
  HB_DDR_WORD_BYTES = 144 /* ABUF / WBUF word in DDR, docs/design.md:402-406 */
};

typedef struct hb_ctx hb_ctx;
typedef struct hb_onchip hb_onchip;

/* GEMM operands, field for field iss::GemmCommand
 * (tools/iss/gemm_array.hpp:16-27; word layout include/hotarubi/isa.hpp:75-94). */
typedef struct hb_gemm_cmd {
  uint32_t a_base, a_stride, kb, m, w_base, w_stride, n8, c_base, wmode, acc;
} hb_gemm_cmd;

/* VEC operands, field for field iss::VecCommand
 * (tools/iss/vec_engine.hpp:70-81). */
typedef struct hb_vec_cmd {
  uint32_t entry, quantize, src, src2, dst, rows_q, n8, p_base, aux, imm;
} hb_vec_cmd;

/* ------------------------------------------------------------ context -- */

/* Version of this ABI (HB_ABI_VERSION). */
int hb_abi_version(void);
/* Message of the calling thread's last failure ("" if none). */
const char* hb_last_error(void);

/* Create a context on HIP device `device` with its own stream. */
int hb_ctx_create(int device, hb_ctx** out);
int hb_ctx_destroy(hb_ctx* ctx);
/* Order the context's work on an existing hipStream_t from now on (NULL is
 * the null stream); the context's own stream, if any, is synchronized and
 * destroyed (so make the first switch before any graph capture: a capture
 * does not allow either).  A context reuses one device workspace across
 * calls (small layers split their K range and finish in a separate
 * element-parallel epilogue), so work issued on an earlier stream must be
 * complete before the switch. */
int hb_ctx_set_stream(hb_ctx* ctx, void* hip_stream);
int hb_ctx_synchronize(hb_ctx* ctx);

/* -------------------------------------------------- on-chip memories -- */

/* Device copies of the on-chip memories, zero-filled
 * (the state of a fresh iss::Memories apart from CBUF, memories.cpp:146-156). */
int hb_onchip_create(hb_ctx* ctx, hb_onchip** out);
int hb_onchip_destroy(hb_onchip* onchip);
/* Copy `count` words starting at word `first` between host and device, in the
 * ISS word layout of `mem` (word sizes above).  first + count <= depth. */
int hb_onchip_upload(hb_onchip* onchip, int mem, uint32_t first,
                     uint32_t count, const void* host);
int hb_onchip_download(hb_onchip* onchip, int mem, uint32_t first,
                       uint32_t count, void* host);
/* Device address of an image, for callers that keep it mirrored themselves. */
int hb_onchip_device_ptr(hb_onchip* onchip, int mem, void** device);

/* ----------------------------------------------- instruction level -- */

/* Decode a 128-bit GEMM instruction word (16 bytes, little-endian) as
 * Machine's DecodeGemm does (tools/iss/machine.cpp:93-104); HB_EINVAL if the
 * opcode field [127:120] is not 4 (GEMM). */
int hb_gemm_decode(const uint8_t word[16], hb_gemm_cmd* out);
/* Encode as EncodeGemm (tools/compiler/isa.cpp:89-103), wait bits 0. */
int hb_gemm_encode(const hb_gemm_cmd* cmd, uint8_t word[16]);
/* The preconditions of ExecuteGemm (gemm_array.cpp:113-119), HB_EBADCMD with
 * the reference's texts; and n8 <= 255, the width of the instruction's n8
 * field (isa.hpp:83), HB_EINVAL otherwise. */
int hb_gemm_check(const hb_gemm_cmd* cmd);
/* Words the instruction reads and writes, one byte per word (1 = touched):
 * reads_abuf[8192], reads_wbuf[2048], reads_fbuf[4096], writes_fbuf[4096];
 * the sets memories.log records (gemm_array.cpp:127,135,141,145), computed on
 * the host so a hazard check needs no device read.  Any pointer may be NULL. */
int hb_gemm_access(const hb_gemm_cmd* cmd, uint8_t* reads_abuf,
                   uint8_t* reads_wbuf, uint8_t* reads_fbuf,
                   uint8_t* writes_fbuf);
/* Execute one GEMM instruction on the device images (exact mode). */
int hb_gemm_exec(hb_ctx* ctx, const hb_gemm_cmd* cmd, hb_onchip* onchip);
int hb_gemm_exec_async(hb_ctx* ctx, const hb_gemm_cmd* cmd, hb_onchip* onchip);
/* Modelled NPU cycles n8*(m/32)*kb*8 + fixed (tools/iss/timing.cpp:65-67,89-93). */
uint64_t hb_gemm_cycles(const hb_gemm_cmd* cmd, uint32_t fixed_cycles);

/* Execute one VEC instruction (VecEngine::Execute, tools/iss/vec_engine.cpp:
 * 157-197) with library entry 0-9 (ADD, MUL, MAX, ADDP, MULP, SCALE, COPY,
 * RELU, ACT, ACT_MUL) or the row programs 12 SOFTMAX, 22 LAYERNORM, 34
 * RMSNORM (tools/compiler/vec_rom.cpp:133-212, 239-272), with or without
 * quantize.  The engine's failures return HB_EBADCMD with its texts.  A row
 * program whose quads touch FBUF or ABUF words that other quads write runs
 * in the engine's pass order (pairs of quads pass by pass, vec_rom.cpp:
 * 84-131) in one workgroup; other row programs run one workgroup per quad.
 * HB_EUNSUPPORTED for other entries (10 ROPE and the transposes). */
int hb_vec_exec(hb_ctx* ctx, const hb_vec_cmd* cmd, hb_onchip* onchip);

/* ---------------------------------------------------- linear level -- */

/* One piece of the fold, LinearPiece (tools/compiler/kernels.hpp:69-74):
 * W blocks [kb_offset, kb_offset + kb).  Its A words: with the descriptor's
 * a_stride 0, the same block indices of A (A is [ceil(m/4)][kb_total]);
 * otherwise block i of quad q is A word q * a_stride + a_word + i (the
 * reference's piece place `a` as a word offset from the descriptor's a, and
 * its a_stride, one stride for all pieces). */
typedef struct hb_piece {
  uint32_t kb_offset; /* first K block of the piece (in W) */
  uint32_t kb;        /* blocks in the piece, >= 1 */
  uint32_t a_word;    /* A word of the piece's first block in quad 0 (a_stride != 0) */
} hb_piece;

/* Epilogue ops, numbered as the VEC library entries (isa.hpp:350-363). */
enum {
  HB_EP_ADDP = 3,  /* y = x + vec[col]        */
  HB_EP_MULP = 4,  /* y = x * vec[col]        */
  HB_EP_SCALE = 5, /* y = x * imm             */
  HB_EP_COPY = 6,  /* y = x (canonicalised)   */
  HB_EP_RELU = 7,  /* y = max(x, 0)           */
  HB_EP_ACT = 8,   /* y = x * T(|x|), SiLU / GELU by the TBUF table */
  HB_EP_ACT_MUL = 9, /* y = ACT(x) * x2[row][col] */
  HB_EP_ADD = 0x100  /* y = x + x2[row][col] (library entry 0, ADD) */
};

typedef struct hb_ep_op {
  uint32_t op;       /* HB_EP_* */
  uint32_t imm;      /* HB_EP_SCALE: the factor as FP32 bits */
  const float* vec;  /* device, n values: HB_EP_ADDP / HB_EP_MULP */
  const float* x2;   /* device, row-major [m][n]: HB_EP_ACT_MUL / HB_EP_ADD */
} hb_ep_op;

/* flags: HB_LINEAR_EXACT or HB_LINEAR_FAST, optionally | HB_LINEAR_PANELS
 * (the W planes are weight panels from hb_pack_weights, not DDR words) or
 * | HB_LINEAR_W8_PANELS (a W8 layer's planes are W8 panels from hb_pack_w8;
 * w[0] and w[1] both point at them); | HB_LINEAR_A_FP8: A holds MXFP8 E4M3
 * codes (hb_encode_mxfp8) instead of MXINT8, against one MXFP4 plane. */
enum {
  HB_LINEAR_EXACT = 0,
  HB_LINEAR_FAST = 1,
  HB_LINEAR_PANELS = 2,
  HB_LINEAR_W8_PANELS = 4,
  HB_LINEAR_A_FP8 = 8
};
enum { HB_MAX_PIECES = 16, HB_MAX_EP_OPS = 8, HB_MAX_GROUP = 4 };

/* C = A x W^T as the emitted instruction sequence computes it:
 *   acc = onto ? c[r][n] : +0
 *   for piece p: for plane l: for block b in piece: acc += BlockValue(...)
 * then ops[0..n_ops) in order, each with the VEC lane formula, then (if
 * q_out) MXINT8 requantization per token and 32 columns.
 *   a       device, MXINT8 DDR words [ceil(m/4)][kb_total] x 144 B (PackAbuf),
 *           or [ceil(m/4)][a_stride] with per-piece offsets (a_stride != 0)
 *   w[l]    device, DDR words [n/8][kb_total] x 144 B (PackWbuf) per plane
 *   modes[l] 0 FP4 (E2M1), 1 W8_HI, 2 W8_LO; a W8 layer is 2 planes {1, 2}
 *   c       device, fp32 row-major [m][n]; read if onto, always written
 *           (4-byte aligned)
 *   q_out   device or NULL, MXINT8 DDR words [ceil(m/4)][n/32] x 144 B
 *           (4-byte aligned)
 *   tbuf    device, 1024 TBUF entries (needed for HB_EP_ACT*)
 * n % 8 == 0 (n % 32 == 0 with q_out); rows of the last quad beyond m are
 * computed from A's rows as given but not stored in c. */
typedef struct hb_linear_desc {
  uint32_t m, n, kb_total;
  uint32_t n_planes;
  uint32_t modes[2];
  const void* a;
  const void* w[2];
  uint32_t n_pieces;
  hb_piece pieces[HB_MAX_PIECES];
  uint32_t onto;
  /* FP32 output [m][n].  May be NULL when q_out is set and onto is 0: the
   * layer then writes only its requantized words, and its FP32 result stays
   * inside the kernel (the NPU keeps it in FBUF and stores only the ABUF
   * words, tools/iss/vec_engine.cpp:447-458).  Not for a layer whose pieces
   * sit at different A offsets (their launches meet in C). */
  float* c;
  uint32_t n_ops;
  hb_ep_op ops[HB_MAX_EP_OPS];
  const uint64_t* tbuf;
  void* q_out;
  /* HB_LINEAR_EXACT: bitwise the NPU's result.  HB_LINEAR_FAST: MXFP4 and
   * W8 layers run on block-scaled matrix cores (exact products, FP32 sums
   * in the hardware's order) and the ops use FP32 hardware arithmetic.
   * Measured bound (every fast-mode parity test checks it; the matrix
   * cores' internal summation order is not documented, so it is not a
   * proof): per element |fast - exact| <= 2^-17 * sum over the folded
   * blocks of |block value| (+ one rounding of each epilogue op), and on
   * N(0,1) activations per output row max |fast - exact| <= 1e-5 *
   * max |exact|.  Tiles whose scale bytes leave the fast path's range are
   * computed exactly.  | HB_LINEAR_PANELS: w[] are weight panels.
   * | HB_LINEAR_W8_PANELS: w[0] = w[1] = W8 panels (one piece over every
   * block; a, w 16-byte aligned); exact mode then folds each output on its
   * own, correct but slow: use DDR words for exact work.
   * | HB_LINEAR_A_FP8 (no counterpart in the reference, which quantizes
   * activations to MXINT8 only): A's 32 code bytes per row and block are
   * OCP E4M3 (E4M3FN; the NaN codes 0x7F / 0xFF are not valid input), its
   * scale bytes E8M0; one MXFP4 plane (modes {0}), DDR words or panels.
   * Exact: each block's exact sum of products, S * 2^-9 * 2^-1 in integer
   * units, is rounded once to FP32 (RNE, below normal -> +0) and the blocks
   * fold as above.  Fast, within the fast-mode bound above (each block's
   * codes go to the FP8 x FP4 matrix cores as two planes split by
   * exponent, so every instruction sums its products without loss): one
   * layer of up to 1,024 rows (ops, requantize, pieces, DDR words or
   * panels); batches of layers of up to 16 rows (the same); batches and
   * larger layers of one piece with the weights in panels (ops and the
   * requantize included).  Other fast MXFP8 layers
   * (batches of more than 16 rows or layers of more than 1,024 rows over
   * DDR words or with several pieces) fold exactly per output (correct,
   * slower). */
  uint32_t flags;
  /* 0: A is [ceil(m/4)][kb_total] words.  Otherwise A words per quad, and
   * each piece's blocks start at its a_word (see hb_piece); every A word a
   * piece reads must lie below byte offset 4 GiB of a. */
  uint32_t a_stride;
} hb_linear_desc;

/* A single small layer (fewer than 128 output tiles) splits its K range
 * over workgroups in the context's workspace, which hb_ctx_create sizes to
 * HB_NOALLOC_SCRATCH_BYTES; a layer that needs more grows it on its first
 * call of that shape (a hipMalloc, with no stream synchronization).  A workspace buffer is never freed before
 * hb_ctx_destroy, so work already queued and HIP graphs captured earlier
 * stay valid when a later call grows it; a graph is valid until its context
 * is destroyed.  Warm a shape up before capturing it in a graph (the
 * allocation itself is not capturable), and do not replay two graphs that
 * use one context's workspace concurrently. */
int hb_linear(hb_ctx* ctx, const hb_linear_desc* desc);
int hb_linear_async(hb_ctx* ctx, const hb_linear_desc* desc);
/* `count` independent layers in one launch (e.g. the same projection of
 * many layers or requests).  Every descriptor must match descs[0] in shape,
 * planes, modes, pieces, onto, flags, TBUF and op kinds/immediates, and each
 * pointer (A, W planes, C, q_out, op vectors) must advance by the same byte
 * stride from one layer to the next; otherwise HB_EINVAL. */
int hb_linear_batched_async(hb_ctx* ctx, const hb_linear_desc* descs,
                            uint32_t count);
/* A group of up to HB_MAX_GROUP layers in one launch where possible (no
 * counterpart in the reference, whose compiler emits each GEMM on its own:
 * the caller knows which of them are independent, e.g. the q, k and v
 * projections of one input).  The result is that of hb_linear_async on
 * each layer in order, provided no layer reads what another writes, with
 * one exception: a layer whose HB_EP_ACT_MUL operand x2 is an earlier
 * layer's c over the same m x n (the gated MLP's gate over up) folds beside
 * it in its workgroups and reads its values there.  Groups of fast
 * layers of at most 160 rows of one weight format (all MXFP4 or all W8 DDR
 * planes, one piece or all several) share one launch; any other group runs
 * as one launch per layer, in order.  No allocation in the shared launch. */
int hb_linear_group_async(hb_ctx* ctx, const hb_linear_desc* descs, uint32_t count);

/* hb_linear_batched_async without any device allocation.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc).  The partial sums and slow flags of a small layer's K splits
 * across workgroups (fast layers of more than 1,024 rows on few tiles, and
 * small exact layers with ops or requantize), which hb_linear keeps in the
 * context's growable workspace, go to a fixed per-device scratch array of
 * HB_NOALLOC_SCRATCH_BYTES instead
 * (resolved when a context is created on the device, held until the
 * process ends).  A layer that needs more returns HB_ENOMEM, naming the
 * size; every other argument rule is hb_linear_batched_async's.  All calls
 * on one GPU share that GPU's array and leave their partials in it:
 * calls that overlap in time on one GPU (different streams or contexts)
 * race, so serialize them. */

#define HB_NOALLOC_SCRATCH_BYTES (8u << 20)
int hb_linear_noalloc_async(hb_ctx* ctx, const hb_linear_desc* descs, uint32_t count);

/* --------------------------------------------------- weight panels -- */

/* Weight panels: a GPU-native layout of one weight plane (no counterpart in
 * the reference, which keeps weights as the DDR words of PackWbuf,
 * tools/compiler/tensors.cpp:66-90).  Packed once per weight, they let the
 * fast kernels stream a column range as one contiguous run instead of 144-byte
 * words of 64 separate column groups; the values are the same codes and scale
 * bytes, so every result (exact and fast) is the one the DDR words give.
 *   n columns (a multiple of 8) x kb_total blocks -> ceil(n / 64) panels of
 *   64 columns; panel p is ceil(kb_total / 2) chunks of 2176 bytes, chunk
 *   (p, s) at byte (p * ceil(kb_total / 2) + s) * 2176, for blocks 2s, 2s + 1:
 *     bytes (b * 64 + c) * 16 .. +15: the 16 code bytes of column 64p + c in
 *       block 2s + b, as in the DDR word (element 2j in the low nibble of
 *       byte j);
 *     byte 2048 + 2 (b * 32 + c % 32) + c / 32: that column-block's E8M0
 *       scale byte.
 *   Columns past n and blocks past kb_total hold zero codes and scale 127.
 * A W8 layer packs each plane (hi, lo) separately.  hb_panel_bytes gives the
 * size of one plane (0 for a bad shape).  hb_pack_weights reads the DDR words
 * [n / 8][kb_total] x 144 B; hb_unpack_weights writes them back bit for bit,
 * with bytes 136..143 of each word (zero in PackWbuf's output) written zero.
 * Both device buffers 16-byte aligned; both calls return when done.  A layer
 * over panels sets HB_LINEAR_PANELS in hb_linear_desc.flags (exact or fast),
 * with w[l] pointing at the panels of plane l. */
uint64_t hb_panel_bytes(uint32_t n, uint32_t kb_total);
int hb_pack_weights(hb_ctx* ctx, const void* w, uint32_t n, uint32_t kb_total, void* panels);
int hb_unpack_weights(hb_ctx* ctx, const void* panels, uint32_t n, uint32_t kb_total, void* w);

/* W8 panels: both nibble planes of a W8 layer (no counterpart in the
 * reference, which keeps them as two WBUF DDR word planes: SplitW8 and
 * PackWbuf, tools/compiler/weights.cpp:72-88, tensors.cpp:66-90) converted
 * once into the FP6 E2M3 operand codes of the GPU's block-scaled matrix
 * cores, so that large-M fast layers convert only A in their K loop.  Each
 * nibble value v (hi plane -8..7, lo plane 0..15) becomes the exact FP6 code
 * of v / 2 and each scale byte ew becomes ew - 1 (hi) or ew - 5 (lo), which
 * the matrix cores' E8M0 scaling turns back into the reference's weights;
 * hb_unpack_w8 restores the DDR words bit for bit.  1.5 bytes per weight
 * (DDR words: 1.125), so skinny layers, bound by weight bandwidth, are
 * better served by DDR words.
 *   n columns (a multiple of 8) x kb_total blocks -> ceil(n / 64) panels of
 *   64 columns, each ceil(kb_total / 2) chunks of 6400 bytes, chunk (p, s)
 *   at (p * ceil(kb_total / 2) + s) * 6400 for blocks 2s + b, b = 0, 1;
 *   with i = (b * 2 + l) * 64 + c for plane l (0 hi, 1 lo), column 64p + c:
 *     bytes i * 16 .. +15 and 4096 + i * 8 .. +7: the column-block's 32 FP6
 *       codes (6 dwords: the first 4, then 2) in the packing of the matrix
 *       cores' FP6 operands (v_cvt_scalef32_pk32_fp6_f16);
 *     byte 6144 + (b * 32 + c % 32) * 4 + 2 (c / 32) + l: its scale byte
 *       minus 1 (hi) or 5 (lo), modulo 256.
 *   Columns past n and blocks past kb_total hold zero codes and scale 127.
 *   Then one dword per panel: nonzero when a scale byte of the panel lies
 *   outside [70, 179] (its tiles are then folded exactly in fast mode).
 * hb_w8_panel_bytes gives the size (0 for a bad shape); hb_pack_w8 reads
 * the hi and lo DDR word planes [n/8][kb_total] x 144 B; hb_unpack_w8 writes
 * them back (bytes 136..143 of each word zero, as PackWbuf writes them).
 * All device buffers 16-byte aligned; both calls return when done. */
uint64_t hb_w8_panel_bytes(uint32_t n, uint32_t kb_total);
int hb_pack_w8(hb_ctx* ctx, const void* w_hi, const void* w_lo, uint32_t n, uint32_t kb_total,
               void* panels);
int hb_unpack_w8(hb_ctx* ctx, const void* panels, uint32_t n, uint32_t kb_total, void* w_hi,
                 void* w_lo);

/* --------------------------------------------- attention W8 operands -- */

/* The DMA engine's on-chip W8 operand builders, over DDR words already in
 * device memory: they make the K and V^T operands of the attention GEMMs
 * (QK^T and PV, tools/compiler/kernels.cpp:155-244) in the W8 plane layout
 * hb_linear takes (modes 1, 2: planes hi then lo).
 *
 * src: `rows` rows of `row_words` MXINT8 words (144 B: 4 tokens x 32 int8,
 * the 4 token scales at byte 128, padding), row r at byte r * src_stride.
 * src, hi, lo 16-byte aligned, src_stride a multiple of 16 (the DMA's beat)
 * and at least row_words * 144, rows and row_words at least 1; otherwise
 * HB_EINVAL.
 *
 * hb_split8 replaces LoadSplit8 (tools/iss/dma_engine.cpp:303-333): rows 2p
 * and 2p + 1 at word position w become plane words (p, w) of hi and lo,
 * [rows/2][row_words] x 144 B each (kb_total = row_words); token j of row
 * 2p + r is column 4r + j, its int8's high nibble goes to hi and low nibble
 * to lo, the token scales are copied, bytes 136..143 are zero.  An odd
 * `rows` returns HB_EBADCMD with the reference's text
 * ("SPLIT8 with an odd number of rows N").
 *
 * hb_t32_split8 replaces LoadT32 / TransposeGroup (dma_engine.cpp:336-398):
 * the planes of the transpose.  Each group of 8 rows (32 tokens) and word
 * position w is a 32 x 32 block; dimension d becomes column d % 8 of column
 * group 4w + d / 8 and the token its K position.  emax is the largest scale
 * among the block's tokens with a nonzero element (127 if none); each
 * element becomes AlignElement(q, emax - e_t) = RNE(q / 2^(emax - e_t)), 0
 * for a shift of 9 or more or an all-zero token (dma_engine.cpp:532-544);
 * all 8 column scales are emax.  hi, lo: [4 * row_words][rows / 8] x 144 B
 * (kb_total = rows / 8).  `rows` not a multiple of 8 returns HB_EBADCMD
 * ("T32_SPLIT8 with N rows, not a multiple of 8").
 *
 * The _async forms are ordered on the context's stream; the others return
 * once the planes are written. */
int hb_split8(hb_ctx* ctx, const void* src, uint64_t src_stride, uint32_t rows,
              uint32_t row_words, void* hi, void* lo);
int hb_split8_async(hb_ctx* ctx, const void* src, uint64_t src_stride, uint32_t rows,
                    uint32_t row_words, void* hi, void* lo);
int hb_t32_split8(hb_ctx* ctx, const void* src, uint64_t src_stride, uint32_t rows,
                  uint32_t row_words, void* hi, void* lo);
int hb_t32_split8_async(hb_ctx* ctx, const void* src, uint64_t src_stride, uint32_t rows,
                        uint32_t row_words, void* hi, void* lo);

/* ----------------------------------------------------- row format -- */

/* The DMA engine's row format for MXINT8 tokens (DMA_LD / DMA_ST of kind
 * ROW and ROW_INDEXED, tools/iss/dma_engine.cpp:96-279; docs/design.md "Row
 * format"): a token is tok blocks of 32 int8, then its tok scale bytes,
 * zero-padded to 16 bytes ((2 tok + (tok > 16 ? 2 : 1)) * 16 bytes); tokens
 * 4q..4q+3 make quad q of the DDR A words hb_linear takes ([quads][tok] x
 * 144 B: bytes 32j.. token j's block, 128 + j its scale, 132..143 zero).
 *
 * hb_row_load replaces LoadRows: rows x row_words tokens, row r at byte
 * r * row_stride of src; or, with index != NULL (ROW_INDEXED, device
 * memory), token e at byte 16 * index[e] of src, 0xFFFFFFFF a zero token
 * (scale bytes 127).  hb_row_store replaces StoreRows (ROW only): the
 * inverse, each token's pad bytes written zero.  The reference's checks
 * return HB_EBADCMD with its texts ("a DMA transfer with R rows of W
 * words", "row format with tok = T", "row format with N tokens, not a
 * multiple of 4", "row format with N tokens of B bytes per row");
 * buffers must be 16-byte aligned and row_stride whole 16-byte beats, at
 * least a row (HB_EINVAL).  FP32 tokens (FBUF) are plain fp32 rows at this
 * level and need no conversion. */
int hb_row_load(hb_ctx* ctx, const void* src, uint64_t row_stride, uint32_t rows,
                uint32_t row_words, uint32_t tok, const uint32_t* index, void* out);
int hb_row_load_async(hb_ctx* ctx, const void* src, uint64_t row_stride, uint32_t rows,
                      uint32_t row_words, uint32_t tok, const uint32_t* index, void* out);
int hb_row_store(hb_ctx* ctx, const void* words, uint32_t rows, uint32_t row_words, uint32_t tok,
                 void* dst, uint64_t row_stride);
int hb_row_store_async(hb_ctx* ctx, const void* words, uint32_t rows, uint32_t row_words,
                       uint32_t tok, void* dst, uint64_t row_stride);

/* ----------------------------------------------------------- GACC -- */

/* The DMA engine's gather-accumulate (DMA_LD of kind GACC, tools/iss/
 * dma_engine.cpp:477-530, 596-656; docs/design.md "GACC"), for `quads`
 * quads at once: quad q's list at list + q * list_stride, 16-byte aligned:
 * a 16-byte header ([31:0] the w area's address) and 16 entries per slot in
 * the order slot s, token t, point k, each [31:0] a row address
 * (0xFFFFFFFF: none), [63:32] bw (FP32).  Addresses count 16-byte units
 * from `base` (device memory holding the rows in MXINT8 row format of
 * `blocks` blocks, and the w areas).  For token t and channel ch, in list
 * order: c = RNE(w[t][ch/32][s] * bw) scaled by 2^(e_row - 6) through the
 * exponent (0 below the normal range, the largest finite value above it),
 * acc = RNE(acc + RNE(int8 * c)); w[t][kb][s] is element t*8 + s%8 of the
 * FBUF word at 16 * (w address + kb * w_stride) + 128 * (s / 8) bytes.
 * out: fp32 [quads * 4][32 * blocks] (token-major rows, the flushed
 * FBUF words' channels); the accumulators start at 0, or at out with
 * accumulate (a chained command with acc = 1).  Bitwise the engine's.
 * The reference's checks return HB_EBADCMD with its texts ("GACC with N
 * blocks per token", "GACC with N slots", "a DMA transfer with 0 rows of
 * N words"). */
typedef struct hb_gacc_desc {
  const void* base;
  const void* list;
  uint64_t list_stride;
  uint32_t quads, slots, blocks, w_stride, accumulate;
  float* out;
} hb_gacc_desc;
int hb_gacc(hb_ctx* ctx, const hb_gacc_desc* desc);
int hb_gacc_async(hb_ctx* ctx, const hb_gacc_desc* desc);

/* --------------------------------------------------- row programs -- */

/* The VEC row programs over row-major tensors in device memory: what
 * hb_vec_exec computes for the same rows laid out as FBUF words (quad q,
 * word w = rows 4q..4q+3, columns 8w..8w+7), with gamma / beta as the PBUF
 * row vectors at p_base / p_base + n8/4.  The producers of a linear layer's
 * A (smolvla_lm.cpp:107-121: RMSNorm + quantize) and the attention softmax.
 *   entry   HB_ROWS_SOFTMAX (12), HB_ROWS_LAYERNORM (22), HB_ROWS_RMSNORM (34)
 *   rows    >= 1; cols a multiple of 8 up to 2040 (n8 = cols/8 <= 255)
 *   x       fp32 [rows][cols]
 *   aux     norms: the element count of the mean (its reciprocal as the
 *           scalar unit's CountReciprocal); softmax: the valid columns
 *   imm     norms: epsilon as FP32 bits
 *   gamma   norms: fp32 [cols]; beta: LAYERNORM, fp32 [cols] (LAYERNORM needs
 *           cols a multiple of 32, where beta's PBUF words follow gamma's)
 *   tbuf    softmax: the TBUF (2^f in entries 0..511)
 *   y       fp32 [rows][cols], or
 *   q_out   MXINT8 DDR words [ceil(rows/4)][cols/32] x 144 B (PackAbuf,
 *           the A of hb_linear); cols a multiple of 32.  Exactly one of y,
 *           q_out.
 * Every buffer is 4-byte aligned (HB_EINVAL otherwise).  Rows of the last
 * quad past `rows` are computed as zero rows (they reach q_out's last words,
 * not y).  Bitwise the NPU's result. */
enum { HB_ROWS_SOFTMAX = 12, HB_ROWS_LAYERNORM = 22, HB_ROWS_RMSNORM = 34 };
typedef struct hb_rows_desc {
  uint32_t entry, rows, cols, aux, imm;
  const float* x;
  const float* gamma;
  const float* beta;
  const uint64_t* tbuf;
  float* y;
  void* q_out;
} hb_rows_desc;
int hb_rows(hb_ctx* ctx, const hb_rows_desc* desc);
int hb_rows_async(hb_ctx* ctx, const hb_rows_desc* desc);

/* --------------------------------------------------------- formats -- */

/* EncodeMxint8 + PackAbuf on device: x fp32 row-major [rows][cols] ->
 * MXINT8 DDR words [ceil(rows/4)][ceil(cols/32)] x 144 B, K zero-padded,
 * rows of the last quad beyond `rows` encoded as zeros.  Inf/NaN input is
 * rejected by the reference (formats.cpp:39); here such an element encodes
 * as 0 and the call returns HB_EINVAL after the launch. */
int hb_encode_mxint8(hb_ctx* ctx, const float* x, uint32_t rows,
                     uint32_t cols, void* out);
/* The MXFP8 E4M3 encoding into the same word layout (no counterpart in the
 * reference): per row and 32-column block, the OCP MX rule -- block
 * exponent floor(log2 max|x|) - 8, clamped to [-127, 127] (0 for a zero
 * block), elements x * 2^-exponent rounded to nearest even on the E4M3
 * grid and saturated to +-448.  Inf/NaN: HB_EINVAL, as hb_encode_mxint8. */
int hb_encode_mxfp8(hb_ctx* ctx, const float* x, uint32_t rows,
                    uint32_t cols, void* out);

/* Weight preparation, the compiler's conversions on device (for a runtime
 * that loads checkpoints straight into GPU memory).  A weight matrix row is
 * an output column of the layer.  Both calls return when done.
 *
 * hb_w8_from_fp32 replaces SplitW8(EncodeMxint8(PadRows(w, out_rows))) and
 * PackWbuf of both planes (tools/compiler/smolvla_common.cpp:95-103,
 * weights.cpp:72-88, tools/runtime/formats.cpp:35-56, tensors.cpp:66-90):
 * fp32 w [rows][cols] -> the W8 layer's hi and lo WBUF word planes
 * [out_rows/8][ceil(cols/32)] x 144 B (modes 1 and 2 of hb_linear_desc).
 * out_rows >= rows and a multiple of 8; rows past `rows` and columns past
 * `cols` are zeros.  Inf/NaN input returns HB_EINVAL (the reference rejects
 * it), after the planes are written with such elements as 0.
 *
 * hb_mxfp4_canonical replaces PackWbuf(CanonicalMxfp4(m, exponent_shift,
 * out_rows)) (weights.cpp:39-70) over the matrix ReadMxfp4 reads
 * (weights.cpp:120-138): codes [rows][cols], one E2M1 code per byte (low
 * nibble), and E8M0 scale bytes [rows][cols/32] -> WBUF words
 * [out_rows/8][cols/32] x 144 B, each block rescaled so its largest code has
 * E2M1 exponent 2.  cols a multiple of 32; out_rows >= rows and a multiple
 * of 8.  A block exponent outside E8M0 returns HB_EINVAL (the reference
 * rejects it), with that scale byte written modulo 256. */
int hb_w8_from_fp32(hb_ctx* ctx, const float* w, uint32_t rows, uint32_t cols,
                    uint32_t out_rows, void* w_hi, void* w_lo);
int hb_mxfp4_canonical(hb_ctx* ctx, const uint8_t* codes, const uint8_t* scales,
                       uint32_t rows, uint32_t cols, int32_t exponent_shift,
                       uint32_t out_rows, void* w);

/* ------------------------------------------------------ DDR images -- */

/* The compiler's DDR image container, DdrImage
 * (tools/compiler/ddr_image.hpp:1-51, ddr_image.cpp:1-63), over device
 * memory: a runtime loads a compiled image (image.bin, and the regions of
 * meta.json, tools/compiler/output.cpp:58-113) into one allocation and takes
 * each named region's device address for hb_linear and the other calls.
 * The region rules are DdrImage's: hb_image_alloc places a region at the
 * image's end rounded up to `align` (0: one page, 4096 bytes) and fails if it
 * passes the capacity; with reuse on, a name already placed returns its
 * region if the size fits (else fails); without reuse, allocating a name
 * again moves it to a new region (one entry, in its first place in the
 * list); hb_image_define names [offset, offset + size) inside the image's
 * end under a new name; hb_image_put writes bytes anywhere below the
 * capacity.  Failures return HB_EINVAL with DdrImage's message.  A new
 * image's bytes are zero.  ctx NULL: bookkeeping only, no device memory
 * (put, get and base are then unavailable). */
typedef struct hb_image hb_image;
int hb_image_create(hb_ctx* ctx, uint64_t capacity, hb_image** out);
void hb_image_destroy(hb_image* image);
int hb_image_alloc(hb_image* image, const char* name, uint64_t size, uint64_t align,
                   uint64_t* offset);
void hb_image_set_reuse(hb_image* image, int reuse);
int hb_image_define(hb_image* image, const char* name, uint64_t offset, uint64_t size);
int hb_image_put(hb_image* image, uint64_t offset, const void* bytes, uint64_t size);
int hb_image_get(const hb_image* image, uint64_t offset, void* bytes, uint64_t size);
int hb_image_region(const hb_image* image, const char* name, uint64_t* offset, uint64_t* size);
uint32_t hb_image_region_count(const hb_image* image);
int hb_image_region_at(const hb_image* image, uint32_t index, const char** name,
                       uint64_t* offset, uint64_t* size);
uint64_t hb_image_end(const hb_image* image);
void* hb_image_base(const hb_image* image);

#ifdef __cplusplus
}
#endif

#endif /* HOTARUBI_GPU_H_ */
