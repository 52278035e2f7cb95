// Internal types shared by the HIP kernels and the C ABI implementation.
//
// Device layout of a quantized weight ("planes"). A GGUF block interleaves
// scales with quants at 34/42/130/144/210-byte strides, which leaves the
// quants 2-byte aligned. At upload every block is split into planes, each a
// [rows][blocks][bytes] array starting on a 256-byte boundary, so that a lane
// loads its quants with 16-byte (dwordx4) loads. The total byte count equals
// the GGUF byte count: the layout moves bytes, it never widens them.
//
//   format   plane 0 (per block)           plane 1            plane 2
//   Q2_0C    128 B codes (bit-permuted)    2 B d (fp16)       -
//   STQ1_0   32 B nibbles (regrouped)      8 B signs (regr.)  2 B d
//   Q4_K     128 B qs (GGUF order)         16 B d,dmin,scales -
//   Q6_K     192 B ql|qh (GGUF order)      16 B int8 scales   2 B d
//   Q8_0     32 B int8 quants              2 B d              -
//   F32/F16  raw values                    -                  -
//
// Q2_0C codes: within each 64-weight unit (16 bytes), device byte 4m+t holds
// in bits 2k..2k+1 the code of weight 16k+4m+t, so that
// (dword_m >> 2k) & 0x03030303 yields the codes of 4 consecutive weights
// 16k+4m..16k+4m+3 (GGUF packs weight i of the unit at byte i/4, bits 2(i%4)).
//
// STQ1_0 nibbles: 16 groups of a 64-weight chunk c occupy 8 bytes; byte
// 8c+4h+t holds group 16c+8h+t in its low nibble and group 16c+8h+4+t in its
// high nibble (the GGUF order is two consecutive groups per byte). Signs: the
// 32 groups of chunks 2j and 2j+1 occupy dword j; bit q+8t is the sign of
// group 16(2j+q/4)+4(q%4)+t, so that (S >> q) & 0x01010101 lines up the signs
// of 4 consecutive groups with 4 bytes.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace hyq {

enum Fmt : int {
    F32 = 0,
    F16 = 1,
    Q8_0 = 8,
    Q4_K = 12,
    Q6_K = 14,
    Q2_0C = 40,
    STQ1_0 = 42
};

// DType::block_len / block_bytes (src/quant.rs:43-62).
inline constexpr int block_len(int f)
{
    return f == F32 || f == F16 ? 1 : f == Q8_0 ? 32 : f == Q2_0C ? 512
           : (f == Q4_K || f == Q6_K || f == STQ1_0) ? 256 : -1;
}
inline constexpr int block_bytes(int f)
{
    return f == F32 ? 4 : f == F16 ? 2 : f == Q4_K ? 144 : f == Q6_K ? 210 : f == Q8_0 ? 34
           : f == Q2_0C ? 130 : f == STQ1_0 ? 42 : -1;
}
// Bytes per block in each device plane.
inline constexpr int plane_bytes(int f, int p)
{
    switch (f) {
    case Q2_0C: return p == 0 ? 128 : p == 1 ? 2 : 0;
    case STQ1_0: return p == 0 ? 32 : p == 1 ? 8 : 2;
    case Q4_K: return p == 0 ? 128 : p == 1 ? 16 : 0;
    case Q6_K: return p == 0 ? 192 : p == 1 ? 16 : 2;
    case Q8_0: return p == 0 ? 32 : p == 1 ? 2 : 0;
    case F32: return p == 0 ? 4 : 0;
    case F16: return p == 0 ? 2 : 0;
    default: return 0;
    }
}
inline constexpr bool is_quant(int f)
{
    return f == Q8_0 || f == Q4_K || f == Q6_K || f == Q2_0C || f == STQ1_0;
}

// A weight (or a view of one expert) on the device: rows x cols, nb blocks
// per row, plane pointers at this view's first row.
struct WView {
    const uint8_t *p0;
    const uint8_t *p1;
    const uint8_t *p2;
    int rows;
    int nb;
};

// Q8 activations on the device (src/quant.rs:861-865) plus integer sums of
// the int8 values over 16-, 32- and 256-element spans (the kernels use them
// to fold the code offsets of Q2_0C, STQ1_0, Q4_K mins and Q6_K's -32).
struct Q8View {
    const int8_t *q;
    const float *s;
    const int32_t *sum16;
    const int32_t *sum32;
    const int32_t *sum256;
    int n;
};

enum GemvMode : int { GEMV_PLAIN = 0, GEMV_SILU = 1, GEMV_MULTI = 2, GEMV_ISUMS = 3 };

struct GemvSeg {
    WView w;
    float *y;
    int row_start; // first row of this segment in the concatenated row space
};

struct GemvArgs {
    GemvSeg seg[3];   // PLAIN/ISUMS: seg[0]; SILU: seg[0]=gate, seg[1]=up; MULTI: up to 3
    int nseg;
    int rows_total;   // rows in the launch's row space
    int groups;       // cols / 256
    Q8View x;
    const float *residual; // PLAIN: y = residual + W x when non-null
    int32_t *isums;        // ISUMS output
    // f32 input stage (decode step): when xin is set, every workgroup forms
    // the Q8 activations of xin itself, in LDS, instead of reading x: of
    // rms_norm(xin) * norm (eps) when norm is set, else of xin.
    const float *xin;
    const float *norm;
    float eps;
    // K split (plain mode with an f32 input stage): kslices > 1 launches
    // kslices workgroup rows; row s covers groups [s*groups, (s+1)*groups) of
    // every matrix row and writes its partial product to
    // seg[0].y + s * rows_total (no residual).
    int kslices;
    // Partial rows (a K split's output) added, in order, to the f32 input of
    // the stage (sparts) and to the residual of the epilogue (rparts):
    // ((v + p[0]) + p[1]) + ... with p[k] = parts + k * parts_stride; at most
    // GEMV_MAX_PARTS of them.
    const float *sparts;
    int nsparts;
    const float *rparts;
    int nrparts;
    int parts_stride;
    // Expert slots (an MoE layer at batch 1): seg[0] (and seg[1]) are stacks
    // of slot_experts experts, and slot_expert[s] (device memory, clamped
    // into range) names the expert of slot s. Row form (nslots == 0): launch
    // row r belongs to slot r / slot_rows and reads row
    // slot_expert[r / slot_rows] * slot_rows + r % slot_rows of the stack;
    // it writes output row r. Slot form (nslots > 0; plain, f32 input stage
    // without norm): workgroup row s is slot s, quantizes its input at
    // xin + s * slot_xin_stride, reads row slot_expert[s] * rows_total + r
    // and writes seg[0].y + s * rows_total.
    const int *slot_expert;
    int slot_experts;
    int slot_rows;
    int nslots;
    int slot_xin_stride;
    // A test hook (the parity tests' record of the int8 codes): with an f32
    // input stage and q8t_codes set, workgroup 0 of each K slice (or slot)
    // writes the f32 values its stage quantized (after the norm), the codes
    // and the scales to q8t_x + 256 * g, q8t_codes + 256 * g and
    // q8t_scales + g for the slice's (slot's) groups g, counted over the
    // launch's K range (slot s: from s * groups).
    int8_t *q8t_codes;
    float *q8t_scales;
    float *q8t_x;
};
constexpr int GEMV_MAX_PARTS = 4;

// Kernel launchers (defined in the .hip files). All return hipError_t as int.
// The Q4_K header plane hdr [rows][nb][16 B] (rows a multiple of 16) copied
// into 16-row tiles [rows / 16][nb][16][16 B] (tiles: rows * nb * 16 bytes).
int launch_tile_headers(const uint8_t *hdr, size_t rows, int nb, uint8_t *tiles, void *stream);
int launch_repack(int fmt, const uint8_t *gguf, size_t nblocks, int nb_per_row, uint8_t *p0,
                  uint8_t *p1, uint8_t *p2, void *stream);
int launch_quantize_q8(const float *x, int n, int8_t *q, float *s, int32_t *sum16,
                       int32_t *sum32, int32_t *sum256, void *stream);
int launch_gemv(int fmt, int mode, const GemvArgs &args, void *stream);
int launch_dequant_rows(int fmt, WView w, int row0, int nrows, int cols, float *out,
                        void *stream);
int launch_decode_gguf(int fmt, const uint8_t *bytes, size_t nblocks, float *out, void *stream);
// Batched products (hyq_gemm.hip): x [rows][K] f32 -> f16 with a power-of-two
// scale per row (rscale), optionally RMS-normalized first (norm [K], eps);
// then the f16-MFMA GEMM
// y[batch][w.rows] = rscale[batch] * (xh[batch][cols] W^T) (+ residual, which
// may alias y), or the dense gate/up product h[batch][gate.rows] =
// silu(gate . x) * (up . x).
// frag: xh in MFMA fragment order (gemm_frag_operand) instead of rows: the
// 8 halves k = 16 b + 8 h .. + 7 of token t at
// ((t / 32 * (K / 16) + b) * 64 + t % 32 + 32 h) * 8, each 32-token block
// (frag_rows: the batch rounded up to whole blocks) one 64 K-byte run.
int launch_to_f16(const float *x, int rows, int K, _Float16 *xh, float *rscale, void *stream,
                  bool frag = false);
inline size_t frag_rows(int batch) { return (size_t)(batch + 31) / 32 * 32; }
// Q8_0 weights at batch 2..FEW_Q80_MAX_TOKENS with cols a multiple of 256
// (hyq_gemm_few.hip): y[n][m] = x[n] . W[m], the activations rounded to f16
// with a power-of-two row scale into xh (few_q80_operand_bytes, in MFMA
// fragment order) and rscale (batch floats), then one product launch with the
// codes exact in the f16 MFMA operands and the block scales applied in f32.
constexpr int FEW_Q80_MAX_TOKENS = 128;
bool few_q80_fits(int rows, int cols, int batch);
size_t few_q80_operand_bytes(int cols, int batch);
int launch_few_q80(WView w, int cols, const float *x, _Float16 *xh, float *rscale, int batch,
                   float *y, void *stream);
int launch_norm_to_f16(const float *x, int rows, int K, const float *norm, float eps,
                       _Float16 *xh, float *rscale, void *stream);
// With `part` (part_floats >= kslices * batch * w.rows) a GEMM of few row
// tiles runs as K slices into part, added in slice order: `kslices` of them,
// or gemm_kslices when kslices is 0.
// xfrag: xh is in fragment order, which only the 256-token tiles take (a
// launch for which gemm_frag_operand holds).
int launch_gemm_f16(int fmt, WView w, int cols, const _Float16 *xh, const float *rscale,
                    int batch, float *y, const float *residual, void *stream,
                    float *part = nullptr, size_t part_floats = 0, int kslices = 0,
                    bool xfrag = false);
// Whether a one-weight product of this shape at `kslices` runs as 256-token
// tiles (and can take its activations in fragment order).
bool gemm_frag_operand(int fmt, int rows, int cols, int batch, int kslices);
int gemm_kslices(int fmt, int M, int K);
size_t gemm_split_floats(int fmt, int M, int N, int K);
int matmul_kslices(int fmt, int M, int K, int batch);
// Up to three weights of one format sharing the activation rows (fused
// Q/K/V): segment i writes y_i [batch][rows_i] (+ residual_i); every segment
// but the last has a multiple of 128 rows. `tiles` is set by the launcher.
struct GemmSeg {
    WView w;
    float *y;
    const float *residual;
    int rows;
    int tiles;
};
struct GemmSegs {
    GemmSeg s[3];
    int nseg;
};
int launch_gemm_f16_segs(int fmt, GemmSegs g, int cols, const _Float16 *xh, const float *rscale,
                         int batch, void *stream, int kslices = 1, float *part = nullptr,
                         bool xfrag = false);
int launch_gate_up_f16(int fmt, WView gate, WView up, int cols, const _Float16 *xh,
                       const float *rscale, int batch, float *h, void *stream);

// Byte offsets of the MoE scratch regions (hyq_gemm.hip: moe_layout).
struct MoeLayout {
    size_t eoff, order, rank, toff, tlist, tiles, ntiles, xg, xscale, h32, h, hscale, outp;
    size_t xop, xhs, xsc, hop, hhs, hsc, cpos, ctok, gpart, upart, xf, bytes;
    int max_tiles, max_tiles_few;
};
MoeLayout moe_layout(int tokens, int npairs, int experts, int hidden, int mid);
int moe_plan_max();
// Expert loop of Moe::forward: gate/up/down are the whole [E] expert stacks.
int launch_moe(int fmt_gu, int fmt_down, WView gate, WView up, WView down, int hidden, int mid,
               const float *x, int tokens, const int *ptok, const int *pexp, const float *pw,
               int npairs, int experts, uint8_t *scratch, const MoeLayout &L, float *out,
               void *stream, const WView *shared = nullptr);
// Whether launch_moe takes a Q8_0 shared projection [hidden, hidden] (`shared`)
// for these shapes: out = x shared^T then the routed sum, the shared product
// run inside the expert launches (the register-operand path with the
// single-workgroup plan, 2..FEW_Q80_MAX_TOKENS tokens).
bool moe_fuses_shared(int fmt_gu, int fmt_down, WView gate, WView up, WView down, int hidden,
                      int mid, int tokens, int npairs, int experts);
// The Q4_K register-operand expert kernels (hyq_moe_q4k.hip) after a plan
// of moe_q4k_chunk()-token chunks. xop/xhs/xsc hold the row operands of the
// token rows of x and hop/hhs/hsc those of the pairs' SiLU rows
// (hyq_moe_operand.hpp), cpos / ctok each chunk column's pair position and
// token (the column's rows), gpart / upart the gate and up partial rows of
// the K slices [2][npairs][mid], outp the down product's rows [npairs][hidden].
// have_ops: the plan's launch already wrote xop/xhs/xsc and cpos/ctok.
// With `shared` (Q8_0, hidden columns, at most FEW_Q80_MAX_TOKENS tokens,
// have_ops, and the plan's launch given xf) the SiLU-rows launch also runs
// y = x shared^T on the f16 fragments xf with the row scales xsc.
int launch_moe_q4k(WView gate, WView up, WView down, int hidden, int mid, const float *x,
                   int tokens, const int *ptok, const int *eoff, const int *valid,
                   const int *order, const int *tiles, const int *ntiles, int max_tiles,
                   int npairs, bool have_ops, uint4 *xop, uint2 *xhs, float *xsc, int *cpos,
                   int *ctok, float *gpart, float *upart, uint4 *hop, uint2 *hhs, float *hsc,
                   float *outp, void *stream, const WView *shared = nullptr,
                   const _Float16 *xf = nullptr, float *y = nullptr);
// whether the register-operand kernels take these expert shapes
bool moe_q4k_fits(int hidden, int mid);
int moe_q4k_chunk();
int isums_per_group(int fmt);
// F32/F16 weights (hyq_f32mm.hip): y[rows] = W x in f32, or silu(W x) *
// (U x) when `up` is given (batch 1); y[batch][rows] = X W^T (batch >= 1).
int launch_f32_gemv(int fmt, WView w, const WView *up, int cols, const float *x, float *y,
                    void *stream);
int launch_f32_gemm(int fmt, WView w, int cols, const float *x, int batch, float *y,
                    void *stream);
// route (hyq_route.hip): per token the `used` experts in ascending index
// with their weights, as slot lists [tokens][used] (slot_expert,
// slot_weight) and, when pair_token is given, the token of each pair.
int route_max_experts();
int launch_route(const float *logits, const float *bias, int tokens, int experts, int used,
                 bool normalize, float scale, int *slot_expert, float *slot_weight,
                 int *pair_token, void *stream);
// out[t] = residual[t] + (shared[t] + w_0 ex[t][0] + ...) in that order
// (without residual: the sum); trace gets a copy when set.
int launch_ffn_combine(const float *residual, const float *shared, const float *ex,
                       const float *w, int used, int H, int tokens, float *out, float *trace,
                       void *stream);
// A read-only stream of `bytes` (16-byte aligned) by `workgroups` workgroups,
// one float per workgroup into sink.
int launch_hbm_read(const void *buf, size_t bytes, int workgroups, float *sink, void *stream);
// `workgroups` x 256 threads issuing `iters` x 4 f16 MFMAs each per wave;
// sink holds workgroups * 256 floats.
int launch_mfma_stream(int workgroups, int iters, float *sink, void *stream);
// rms_norm_into of `rows` rows of width H into y (f32).
int launch_rms_rows(const float *x, const float *w, int rows, int H, float eps, float *y,
                    void *stream);

} // namespace hyq
