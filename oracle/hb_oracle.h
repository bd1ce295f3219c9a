/*
 * CPU oracle for the quantized GEMM hot path (test infrastructure only).
 *
 * This is a plain-C restatement of the reference CPU path: the ISS GEMM
 * instruction (tools/iss/gemm_array.cpp), its FP32 arithmetic
 * (tools/iss/fp32.hpp), the operand formats and packers
 * (tools/runtime/formats.cpp, tools/compiler/tensors.cpp,
 * tools/compiler/weights.cpp), the VEC epilogue subset
 * (tools/iss/lane.cpp, tools/iss/vec_engine.cpp, tools/compiler/vec_rom.cpp)
 * and the fold order of an emitted linear layer
 * (tools/compiler/kernels.cpp:343-395).
 *
 * Only the tests, the smoke check and the CPU-baseline leg of the benchmark
 * load this library, and only as the checker.  The product library
 * (libhotarubi_gpu.so) never links or calls it.
 *
 * The MXFP8 functions restate no reference code (the reference has no FP8
 * activation format); they are this build's definition of that extension.
 *
 * Every function here is pinned by at least one of: the reference's own
 * known-answer tests (tests/golden/), the reference FP32 sources compiled
 * from /root/reference into oracle/_ref, closed-form checks in
 * tests/test_oracle_*.py (exact rational arithmetic, brute force on tiny
 * inputs, invariants).  No function is "parity unpinned".
 */
#ifndef HB_ORACLE_H_
#define HB_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* On-chip memory geometry (tools/iss/memories.hpp:16-34). */
enum {
  HBO_TOKENS = 4,
  HBO_LANES = 8,
  HBO_BLOCK = 32,
  HBO_ABUF_WORD = 132, /* in-ISS word: 128 int8 + 4 scales */
  HBO_WBUF_WORD = 144, /* 128 nibble bytes + 8 scales + 8 pad */
  HBO_DDR_WORD = 144,  /* ABUF/WBUF word in DDR (docs/design.md:402-406) */
  HBO_ABUF_DEPTH = 8192,
  HBO_WBUF_DEPTH = 2048,
  HBO_FBUF_DEPTH = 4096,
  HBO_PBUF_DEPTH = 512,
  HBO_TBUF_DEPTH = 1024
};

/* Mirrors iss::GemmCommand (tools/iss/gemm_array.hpp:16-27). */
typedef struct {
  uint32_t a_base, a_stride, kb, m, w_base, w_stride, n8, c_base, wmode, acc;
} hbo_gemm_cmd;

/* Mirrors iss::VecCommand (tools/iss/vec_engine.hpp:70-81). */
typedef struct {
  uint32_t entry, quantize, src, src2, dst, rows_q, n8, p_base, aux, imm;
} hbo_vec_cmd;

/* Last error message of the calling thread ("" if none). */
const char* hbo_last_error(void);

/* ---- FP32 semantics: tools/iss/fp32.hpp:24-104 ---- */
uint32_t hbo_fp32_pack(uint32_t sign, int32_t exponent, uint32_t fraction);
uint32_t hbo_fp32_round(uint32_t sign, int32_t exponent, uint32_t significand,
                        int guard, int sticky);
uint32_t hbo_fp32_add(uint32_t a, uint32_t b);
uint32_t hbo_fp32_mul(uint32_t a, uint32_t b);
uint32_t hbo_fp32_mul_fraction(uint32_t s, uint32_t fraction);

/* ---- GEMM array: tools/iss/gemm_array.cpp ---- */
uint32_t hbo_decode_weight_mode(uint32_t wmode);          /* :73-82 */
int32_t hbo_weight_value(uint32_t nibble, uint32_t mode); /* :84-97 */
int32_t hbo_scale_bias(uint32_t mode);                    /* :25-35 */
uint32_t hbo_block_value(int32_t sum, uint32_t a_scale, uint32_t w_scale,
                         uint32_t mode); /* :99-110 */
/* ExecuteGemm (:112-149) on ISS-layout images:
 * abuf[8192][132], wbuf[2048][144], fbuf[4096][32].  Returns 0 on success,
 * nonzero (message in hbo_last_error) when the preconditions of :113-119
 * fail; the images are then untouched. */
int hbo_gemm_exec(const hbo_gemm_cmd* cmd, const uint8_t* abuf,
                  const uint8_t* wbuf, uint32_t* fbuf);
/* Access sets of ExecuteGemm (memories.log reads/writes at :127,135,141,145)
 * as one byte per word: reads_abuf[8192], reads_wbuf[2048], reads_fbuf[4096],
 * writes_fbuf[4096] (1 = accessed). */
int hbo_gemm_access(const hbo_gemm_cmd* cmd, uint8_t* reads_abuf,
                    uint8_t* reads_wbuf, uint8_t* reads_fbuf,
                    uint8_t* writes_fbuf);

/* ---- formats: tools/runtime/formats.cpp ---- */
int8_t hbo_quantize_int8(uint32_t bits, int32_t e); /* :35-56 */
/* EncodeMxint8 (:138-162): x row-major [rows][cols] fp32 bits ->
 * q [rows][kpad] int8, e [rows][kpad/32] int32, kpad = PadToBlock(cols). */
int hbo_encode_mxint8(const uint32_t* x, uint32_t rows, uint32_t cols,
                      int8_t* q, int32_t* e);
/* PackAbuf (:114-136): q [rows][cols], e [rows][cols/32] -> DDR words
 * [(rows/4) * (cols/32)][144]. */
int hbo_pack_abuf(const int8_t* q, const int32_t* e, uint32_t rows,
                  uint32_t cols, uint8_t* out);
/* PackFbuf / UnpackFbuf (:72-112): row-major [rows][cols] <-> words. */
int hbo_pack_fbuf(const uint32_t* x, uint32_t rows, uint32_t cols,
                  uint32_t* out);
int hbo_unpack_fbuf(const uint32_t* words, uint32_t rows, uint32_t cols,
                    uint32_t* out);

/* ---- weights: tools/compiler/tensors.cpp:66-90, weights.cpp:39-88 ---- */
/* PackWbuf: code [rows][cols] (low 4 bits used), e [rows][cols/32] ->
 * DDR words [(rows/8) * (cols/32)][144]. */
int hbo_pack_wbuf(const uint8_t* code, const int32_t* e, uint32_t rows,
                  uint32_t cols, uint8_t* out);
/* SplitW8: q -> hi = byte >> 4, lo = byte & 15 (scales shared). */
void hbo_split_w8(const int8_t* q, size_t count, uint8_t* hi, uint8_t* lo);
/* CanonicalMxfp4 (weights.cpp:39-70), out has out_rows >= rows rows. */
int hbo_canonical_mxfp4(const uint8_t* code, const int32_t* e, uint32_t rows,
                        uint32_t cols, int32_t exponent_shift,
                        uint32_t out_rows, uint8_t* out_code, int32_t* out_e);

/* ---- VEC lane: tools/iss/lane.cpp ---- */
uint32_t hbo_interpolate(uint64_t entry, uint32_t fraction);       /* :337 */
uint32_t hbo_activation(uint32_t prod, const uint64_t* tbuf);       /* :342 */
uint32_t hbo_post_add(uint32_t prod, uint32_t c1, uint32_t op);     /* :322 */
uint8_t hbo_quantize_element(uint32_t value, uint32_t emax);        /* :384 */
int hbo_quantize_block(const uint32_t* words4x32, uint8_t* out132); /* :406 */

/* ---- row reductions: tools/iss/scalar.cpp, lane.cpp:67-99, 357-382 ---- */
uint32_t hbo_reciprocal(uint32_t bits);                  /* scalar.cpp:44 */
uint32_t hbo_rsqrt(uint32_t bits);                       /* scalar.cpp:54 */
uint32_t hbo_count_reciprocal(uint32_t count);           /* scalar.cpp:64 */
uint32_t hbo_sum_tree(const uint32_t* v8);               /* scalar.cpp:26 */
uint32_t hbo_max_tree(const uint32_t* v8);               /* scalar.cpp:32 */
uint32_t hbo_fp32_max(uint32_t a, uint32_t b);           /* lane.cpp:380 */
uint32_t hbo_exp2(uint32_t prod, const uint64_t* tbuf);  /* lane.cpp:357 */
/* LaneOutput for the row programs' pass fields: c0 0 zero, 1 rs0, 2 pbuf;
 * b 0 one, 1 pre, 2 rs1, 3 pbuf, 4 imm; nl 1 Exp2; cmp 1 (w*8+l) < imm2;
 * sel 0 none, 1 zero, 2 null (lane.cpp:163-179, 281-320). */
uint32_t hbo_row_lane(int c0, int b, int nl, int cmp, int sel, uint32_t x, uint32_t pbuf,
                      uint32_t t, uint32_t l, uint32_t w, uint32_t imm, uint32_t imm2,
                      uint32_t rs0, uint32_t rs1, const uint64_t* tbuf);
/* ApplyRowScalar (scalar.cpp:71-97): red 1 sum, 2 max; sf 1 negate, 2
 * reciprocal, 3 rsqrt, 4 identity; sum [4][8], max [4] -> out [4]. */
void hbo_apply_row_scalar(int red, int sf, int st, int srn, int seps, const uint32_t* sum,
                          const uint32_t* max, uint32_t epsilon, uint32_t rn, uint32_t* out);

/* VecEngine::Execute for library entries 0-9 (ADD, MUL, MAX, ADDP, MULP,
 * SCALE, COPY, RELU, ACT, ACT_MUL) and the row programs 12 (SOFTMAX), 22
 * (LAYERNORM) and 34 (RMSNORM), with and without quantize.  Images in ISS
 * layout: abuf[8192][132], fbuf[4096][32], pbuf[512][32], tbuf[1024].
 * Returns nonzero (and leaves the images in an unspecified state) where the
 * reference calls Fail; 2 for other entries. */
int hbo_vec_exec(const hbo_vec_cmd* cmd, uint8_t* abuf, uint32_t* fbuf,
                 const uint32_t* pbuf, const uint64_t* tbuf);

/* ---- row format (DMA ROW / ROW_INDEXED, MXINT8): dma_engine.cpp:96-279 ---- */
/* Token bytes (2 tok + (tok > 16 ? 2 : 1)) * 16.  Load: rows x row_words
 * tokens (row r at r * row_stride bytes) or, with index, token e at byte
 * 16 * index[e] of src (0xFFFFFFFF: a zero token, scale bytes 127) -> DDR A
 * words [tokens/4][tok] x 144 B.  Store: the inverse, pad bytes zero.
 * Nonzero with the reference's text on a rejected shape. */
uint32_t hbo_row_token_bytes(uint32_t tok);
int hbo_row_load(const uint8_t* src, uint64_t row_stride, uint32_t rows, uint32_t row_words,
                 uint32_t tok, const uint32_t* index, uint8_t* out);
int hbo_row_store(const uint8_t* words, uint32_t rows, uint32_t row_words, uint32_t tok,
                  uint8_t* dst, uint64_t row_stride);

/* ---- GACC gather-accumulate: dma_engine.cpp:477-530, 596-656 ---- */
uint32_t hbo_int8_to_fp32(uint8_t value);
uint32_t hbo_scale_coefficient(uint32_t coefficient, uint32_t scale);
/* One quad: base = DDR byte 0 (16-byte unit addresses), list = the quad's
 * list (header: w area address; entries [row address, bw] in order s, t, k),
 * w_stride the w areas' block stride in 16-byte units; acc [4][32*blocks]. */
int hbo_gacc(const uint8_t* base, const uint8_t* list, uint32_t slots, uint32_t blocks,
             uint32_t w_stride, int accumulate, uint32_t* acc);

/* ---- linear layer: tools/compiler/kernels.cpp:343-395 ---- */
enum { HBO_EP_NONE = 0, HBO_EP_ADDP = 3, HBO_EP_MULP = 4, HBO_EP_SCALE = 5,
       HBO_EP_COPY = 6, HBO_EP_RELU = 7, HBO_EP_ACT = 8, HBO_EP_ACT_MUL = 9,
       HBO_EP_ADD = 0x100 };

typedef struct {
  uint32_t op;          /* HBO_EP_* (library entry numbers) */
  uint32_t imm;         /* SCALE factor bits */
  const uint32_t* vec;  /* ADDP/MULP: n fp32 bits, one per column */
  const uint32_t* x2;   /* ACT_MUL (up) / ADD (residual): [m][n] fp32 bits */
} hbo_ep_op;

typedef struct {
  uint32_t kb_offset, kb;
} hbo_piece;

/* One linear layer as the emitted GEMM sequence computes it: per output,
 *   acc = onto ? c[r][n] : +0
 *   for piece p: for plane l: for block b: acc = Add(acc, BlockValue(...))
 * then the epilogue ops in order (each with the VEC lane formula), then
 * optionally QuantizeBlock per 4 tokens x 32 columns.
 *   a      : A DDR words [(m/4)][kb_total][144] (PackAbuf layout)
 *   w[l]   : plane l DDR words [(n/8)][kb_total][144] (PackWbuf layout)
 *   modes[l]: 0 FP4, 1 W8_HI, 2 W8_LO
 *   c      : fp32 bits row-major [m][n] (input if onto, output always)
 *   q_out  : if non-NULL, MXINT8 DDR words [(m/4)][(n/32)][144]
 * m must be a multiple of 4, n of 8 (of 32 with q_out). */
int hbo_linear(uint32_t m, uint32_t n, uint32_t kb_total, const uint8_t* a,
               uint32_t n_planes, const uint8_t* const* w,
               const uint32_t* modes, uint32_t n_pieces,
               const hbo_piece* pieces, int onto, uint32_t* c,
               uint32_t n_ops, const hbo_ep_op* ops, const uint64_t* tbuf,
               uint8_t* q_out);

/* MXFP8 E4M3 activations (no counterpart in the reference; this build's
 * definition, see hb_oracle.c): E4M3 code -> integer in units of 2^-9, the
 * block value of S = sum A_int * W_int rounded once to FP32, the OCP MX
 * encoder, and the linear fold over one MXFP4 weight plane. */
int32_t hbo_fp8_int(uint8_t code);
uint32_t hbo_block_value_fp8(int32_t sum, uint32_t a_scale, uint32_t w_scale);
uint8_t hbo_quantize_fp8(uint32_t bits, int32_t x);
int hbo_encode_mxfp8(const uint32_t* x, uint32_t rows, uint32_t cols, uint8_t* q,
                     int32_t* e);
int hbo_linear_fp8(uint32_t m, uint32_t n, uint32_t kb_total, const uint8_t* a,
                   const uint8_t* w, uint32_t n_pieces, const hbo_piece* pieces, int onto,
                   uint32_t* c, uint32_t n_ops, const hbo_ep_op* ops, const uint64_t* tbuf,
                   uint8_t* q_out);

/* Batched forms for the tests. */
void hbo_fp32_add_n(const uint32_t* a, const uint32_t* b, uint32_t* out, uint64_t n);
void hbo_fp32_mul_n(const uint32_t* a, const uint32_t* b, uint32_t* out, uint64_t n);
void hbo_fp32_mul_fraction_n(const uint32_t* s, const uint32_t* f, uint32_t* out,
                             uint64_t n);
void hbo_block_value_n(const int32_t* sum, const uint32_t* a_scale,
                       const uint32_t* w_scale, uint32_t mode, uint32_t* out,
                       uint64_t n);

/* On-chip W8 operand builders of the DMA engine, over DDR words.
 * src: `rows` rows of `row_words` MXINT8 words (144 B: 4 tokens x 32 int8,
 * 4 scale bytes at 128, pad), row r at byte r * src_stride.
 *
 * SPLIT8 (LoadSplit8, tools/iss/dma_engine.cpp:303-333): rows 2p and 2p+1
 * at word position w give W8 plane words (p, w): token j of row 2p + r is
 * column 4r + j; high nibbles to `hi`, low nibbles to `lo`, token scales
 * copied.  hi / lo: [rows/2][row_words] 144-byte words (bytes 136..143 0).
 *
 * T32_SPLIT8 (TransposeGroup / LoadT32, dma_engine.cpp:336-398): each group
 * of 8 rows (32 tokens) and word position w is transposed: dimension d is
 * column d % 8 of column group 4w + d / 8, the token its K position, with
 * the tokens' scales aligned to emax (the largest scale among tokens with a
 * nonzero element, 127 if none): element = AlignElement(q, emax - e_t), 0
 * for an all-zero token.  hi / lo: [4 * row_words][rows / 8] words.
 *
 * AlignElement (dma_engine.cpp:532-544): RNE(q / 2^shift) as a byte, 0 for
 * shift >= 9. */
uint8_t hbo_align_element(uint8_t value, uint32_t shift);
int hbo_split8(const uint8_t* src, uint64_t src_stride, uint32_t rows,
               uint32_t row_words, uint8_t* hi, uint8_t* lo);
int hbo_t32_split8(const uint8_t* src, uint64_t src_stride, uint32_t rows,
                   uint32_t row_words, uint8_t* hi, uint8_t* lo);

/* GEMM cost model (tools/iss/timing.cpp:65-67,89-93), cycles at 250 MHz. */
uint64_t hbo_gemm_cycles(const hbo_gemm_cmd* cmd, uint32_t fixed_cycles);

#ifdef __cplusplus
}
#endif

#endif /* HB_ORACLE_H_ */
