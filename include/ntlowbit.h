/*
 * ntlowbit.h: C-ABI of the MI355X (gfx950) low-bit linear hot path.
 *
 * One shared library, libntlowbit.so, built from nano-train_amd/csrc/.  The
 * signatures hold only plain pointers, integers and an opaque stream handle
 * (a hipStream_t passed as void*, NULL = the null stream), so any FFI can
 * bind them.  All device pointers are caller-allocated; no entry point
 * allocates, frees or synchronizes.  Every launch is asynchronous on `stream`.
 *
 * Each entry point replaces one torch-op sequence of nano-train's emulated
 * backend; the reference function it stands in for is cited as
 * path:line into lastweek/nano-train.
 *
 * Return values: NTLB_OK (0) on success, a negative NTLB_E* status otherwise;
 * ntlb_last_error() then describes the failure (thread-local string).
 *
 * Conventions
 *   dtype   : NTLB_F32, NTLB_BF16, NTLB_F16 for float tensors.
 *   grid    : NTLB_GRID_INT  - int8 codes of the reference's symmetric integer
 *                              grid, |q| <= qmax = 2^(bits-1)-1, scale =
 *                              amax/qmax (te_backend.py:98-106); a NaN element
 *                              is stored as code -128;
 *             NTLB_GRID_E4M3 - OCP e4m3fn codes, scale = amax/448 (the
 *                              DeepSeek-V3 recipe).
 *   rounding: NTLB_ROUND_NEAREST (torch.round, half to even) or
 *             NTLB_ROUND_STOCHASTIC: element e uses r = word e%4 of
 *             Philox4x32-10(counter {lo(e/4), hi(e/4), lo(offset), hi(offset)},
 *             key {lo(seed), hi(seed)}).  Int grid: u = (r >> 8) * 2^-24,
 *             and v rounds to floor(v+u) for v >= 0, ceil(v-u) for v < 0
 *             (te_backend.py:61-65).  e4m3: |v| rounds away from zero exactly
 *             when f + (r >> 12) >= 2^20, f being the 20 bits of |v|'s
 *             significand below the e4m3 spacing (for subnormal results, of
 *             |v| * 512 below its integer part): gfx950's v_cvt_sr_fp8_f32.
 *             e is the row-major index of the element in the source matrix.
 *   codes   : uint8 [rows, ldc], ldc >= ceil(K/128)*128 where tiles pad K;
 *             padding columns are written as 0.
 *   scales  : fp32; element (i, t) lives at scales[i*s_row + t*s_col], so
 *             either layout (row-major or tile-major) can be requested.
 */
#ifndef NTLOWBIT_H
#define NTLOWBIT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NTLB_ABI_VERSION 1

#define NTLB_OK 0
#define NTLB_EINVAL (-1)       /* bad shape, stride, alignment or enum */
#define NTLB_ELAUNCH (-2)      /* the HIP runtime refused a launch */
#define NTLB_EUNSUPPORTED (-3) /* valid request this build does not cover */

#define NTLB_F32 0
#define NTLB_BF16 1
#define NTLB_F16 2

#define NTLB_GRID_INT 0
#define NTLB_GRID_E4M3 1

#define NTLB_ROUND_NEAREST 0
#define NTLB_ROUND_STOCHASTIC 1

/* scale rules: te_backend.py:74-79 (safe(amax/qmax)) and moe.py:94-98
 * (amax checked before the division) */
#define NTLB_SCALE_AFTER_DIVIDE 0
#define NTLB_SCALE_BEFORE_DIVIDE 1

int ntlb_abi_version(void);
const char* ntlb_last_error(void);

/*
 * 1x128 tile quantizer.  Replaces _tile_quant_dequant (te_backend.py:82-110)
 * and the tile_1x128 branch of _quantize_dequantize_with_granularity
 * (te_backend.py:187-193).
 *   x      [R, K] with row stride ldx (elements), last dim contiguous.
 *   codes  [R, ldc] uint8, ldc >= ceil(K/128)*128, multiple of 8.
 *   scales [R, T] (T = ceil(K/128)) addressed with (s_row, s_col).
 *   dq     optional [R, K] (row stride lddq) = q*scale cast to dq_dtype
 *          (the tensor the reference returns); NULL to skip.
 *   nan_rows optional int32 [R]: rows holding a NaN get 1 OR-ed in; the
 *          caller zeroes it.  NULL to skip.
 */
int ntlb_quant_tile_1x128(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int grid, int qmax,
                          int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* codes,
                          int64_t ldc, float* scales, int64_t s_row, int64_t s_col, void* dq, int dq_dtype,
                          int64_t lddq, int32_t* nan_rows, void* stream);

/*
 * ntlb_quant_tile_1x128 of the token rows gathered by expert: the gather
 * tokens[token_indices] of the per-expert loop (moe.py:1081, :484) fused into
 * the quantizer.  Token row r of x [T, K] (row stride ldx) becomes output row
 * pos[r*fan_k + f] for f < fan_k (pos from ntlb_ep_partition on topk_idx
 * [T, fan_k] with divisor 1 and one bucket per expert), each token row read
 * once.  Codes, scales (s_row, s_col), nan_rows and the SR element index
 * (p*K + column) are those ntlb_quant_tile_1x128 writes for row p of the
 * gathered matrix [rows, K], bit for bit.  A negative pos entry (an
 * assignment a capacity limit dropped) writes nothing, and output rows that
 * no entry names are left as they are; entries at or past rows are clamped
 * to rows - 1.  x bf16 or fp32, K % 8 == 0, 16-byte aligned rows, codes
 * 8-byte aligned, ldc >= ceil(K/128)*128 and a multiple of 8.
 */
int ntlb_quant_tile_1x128_fanout(const void* x, int x_dtype, int64_t T, int64_t K, int64_t ldx, const int32_t* pos,
                                 int64_t fan_k, int64_t rows, int grid, int qmax, int rounding, int scale_rule,
                                 uint64_t seed, uint64_t offset, uint8_t* codes, int64_t ldc, float* scales,
                                 int64_t s_row, int64_t s_col, int32_t* nan_rows, void* stream);

/*
 * 128x128 block quantizer for a 2-D weight.  Replaces _block_quant_dequant
 * (te_backend.py:113-149).
 *   w [N, K] (row stride ldw); codes [N, ldc]; scales [ceil(N/128), T] via
 *   (s_row, s_col); optional transposed codes codes_t [K, ldct] (ldct >=
 *   ceil(N/128)*128) for GEMMs that contract over N; optional dq and
 *   nan_rows as for the tile quantizer.
 */
int ntlb_quant_block_128x128(const void* w, int w_dtype, int64_t N, int64_t K, int64_t ldw, int grid, int qmax,
                             int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* codes,
                             int64_t ldc, uint8_t* codes_t, int64_t ldct, float* scales, int64_t s_row,
                             int64_t s_col, void* dq, int dq_dtype, int64_t lddq, int32_t* nan_rows, void* stream);

/*
 * Grouped amax: amax_bits[(i/gr)*n_gc + k/gc] = max |x[i,k]| as fp32 bits
 * (NaN-propagating).  The caller zeroes amax_bits.  Together with
 * ntlb_quant_grouped this covers the granularities whose groups span many
 * rows: tensor (gr=R, gc=K; te_backend.py:165-173), channel along the last
 * axis (gr=R, gc=1) or axis 0 (gr=1, gc=K) (te_backend.py:175-185), and the
 * comm-quant strip (gr=R, gc=128; moe.py:123-140).
 */
int ntlb_amax_grouped(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr, int64_t gc,
                      uint32_t* amax_bits, void* stream);

/*
 * _comm_quant_dequant (moe.py:79-143) in one pass: x [R, K] quantized with one
 * scale per (gr x gc) group (scales from the amaxes of ntlb_amax_grouped,
 * scale_rule, qmax and grid as in ntlb_quant_grouped; the reference uses
 * the int grid, qmax 2^(bits-1)-1 and NTLB_SCALE_BEFORE_DIVIDE), and out
 * [R, ldo] (x's dtype) = the value the reference returns, tensor + (dq -
 * tensor) evaluated in x's dtype with dq = q * scale rounded to that dtype.
 * Granularities: tile_1x128 / block_128x128 (gr = R, gc = 128), channel
 * (gr = R, gc = 1), tensor (gr = R, gc = K).  Autograd (the straight-through
 * gradient) stays with the caller.
 */
int ntlb_comm_quant_dequant(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr, int64_t gc,
                            const uint32_t* amax_bits, int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                            uint64_t offset, void* out, int64_t ldo, void* stream);

/*
 * Quantize with precomputed group amaxes (from ntlb_amax_grouped).  Writes
 * scales[(i/gr)*n_gc + k/gc] (fp32, computed from the amax with scale_rule),
 * codes [R, ldc] (ldc >= K), optional dq and nan_rows.
 */
int ntlb_quant_grouped(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr, int64_t gc,
                       const uint32_t* amax_bits, int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                       uint64_t offset, uint8_t* codes, int64_t ldc, float* scales, void* dq, int dq_dtype,
                       int64_t lddq, int32_t* nan_rows, void* stream);

/*
 * ntlb_amax_grouped followed by ntlb_quant_grouped without the amax
 * workspace.  It has no counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and outputs as
 * ntlb_quant_grouped minus amax_bits (the caller still passes x, codes,
 * scales and the optional dq and nan_rows).  The group amaxes accumulate in a
 * file-scope device array of 65536 words (256 KiB on each GPU the library
 * runs on, held until the process ends), cleared by a kernel at the start of
 * every call; more than 65536 scale groups (ceil(R/gr) * ceil(K/gc)) is
 * NTLB_EINVAL.  Every call on a GPU shares that GPU's array: calls that may
 * overlap on one GPU (different streams) race.  Allocates nothing.
 */
int ntlb_quant_grouped_noalloc(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int64_t gr, int64_t gc,
                               int grid, int qmax, int rounding, int scale_rule, uint64_t seed, uint64_t offset,
                               uint8_t* codes, int64_t ldc, float* scales, void* dq, int dq_dtype, int64_t lddq,
                               int32_t* nan_rows, void* stream);

/*
 * 128x1 tile quantizer with transposed codes: groups of 128 consecutive rows
 * of one column share a scale, and the codes are written transposed,
 * codes_t [K, ldct] (ldct >= ceil(R/128)*128, a multiple of 16).  These are
 * the contraction-over-tokens operands X^T and dY^T of the DeepSeek-V3 wgrad
 * recipe; there is no reference function (te_backend.py:250-260 leaves dY
 * unquantized).  It is _tile_quant_dequant (te_backend.py:82-110) applied to
 * x^T.  scales(k, mb) = scales[k*s_row + mb*s_col].  SR bits are keyed by the
 * source index r*K + k.  Optional dq [R, K] as above; optional nan_rows [K] has
 * one flag per transposed row (source column k), set when a NaN reached it.
 */
int ntlb_quant_tile_128x1_t(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int grid, int qmax,
                            int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* codes_t,
                            int64_t ldct, float* scales, int64_t s_row, int64_t s_col, void* dq, int dq_dtype,
                            int64_t lddq, int32_t* nan_rows, void* stream);

/*
 * Dual-output pass for a gradient dY: one read of x [R, K] writes both its
 * 1x128 tiles (codes [R, ldc], scales addressed (s_row, s_col), nan_rows [R],
 * SR offset offset_rows) -- exactly ntlb_quant_tile_1x128 -- and its 128x1
 * tiles with transposed codes (codes_t [K, ldct], scales_t addressed
 * (st_row, st_col), nan_cols [K], SR offset offset_cols) -- exactly
 * ntlb_quant_tile_128x1_t.  These are the dgrad and wgrad operands of the
 * DeepSeek-V3 recipe backward; there is no reference function (the reference
 * backward, te_backend.py:250-260, leaves dY unquantized), and each output
 * follows _tile_quant_dequant (te_backend.py:82-110) as its single-output
 * entry point does.  Needs bf16 or fp32 x, K % 8 == 0, ldx % 8 == 0 and
 * 16-byte aligned rows (NTLB_EUNSUPPORTED otherwise: use the two entry points).
 */
int ntlb_quant_dual_1x128_128x1(const void* x, int x_dtype, int64_t R, int64_t K, int64_t ldx, int grid, int qmax,
                                int rounding, int scale_rule, uint64_t seed, uint64_t offset_rows,
                                uint64_t offset_cols, uint8_t* codes, int64_t ldc, float* scales, int64_t s_row,
                                int64_t s_col, int32_t* nan_rows, uint8_t* codes_t, int64_t ldct, float* scales_t,
                                int64_t st_row, int64_t st_col, int32_t* nan_cols, void* stream);

/*
 * Dequantize codes back to a float tensor: out[i, k] = q(code) * scale(i, k)
 * with scale(i, k) = scales[(i >> r_shift) * s_row + (k >> c_shift) * s_col]
 * (shifts 0 or 7; a zero stride broadcasts), cast to out_dtype.  The receive
 * side of the comm-quant wire format (the receiver's .to(tokens.dtype) of
 * moe.py:822-823, :998-999) and the dq of any quantizer above.
 */
int ntlb_dequant(int grid, const uint8_t* codes, int64_t ldc, const float* scales, int64_t s_row, int64_t s_col,
                 int r_shift, int c_shift, int64_t R, int64_t K, void* out, int out_dtype, int64_t ldo,
                 void* stream);

/*
 * Blockwise-scaled GEMM  Y[M,N] = sum_kb sa(m,kb) * sb(n,kb) * (A_kb[m,:] . B_kb[n,:])  (+ bias[n]).
 * The math of F.linear(X_dq, W_dq, bias) in te_backend.py:253-259 with the
 * operands kept as codes plus scales: every 128-wide K block is multiplied
 * on the matrix cores (int8 MFMA for NTLB_GRID_INT, fp8 e4m3 MFMA for
 * NTLB_GRID_E4M3) and promoted into an fp32 accumulator with its scales.
 *   a  [M, Kp] codes, row stride lda;  b [N, Kp] codes, row stride ldb;
 *      Kp a multiple of 128, lda/ldb multiples of 16, 16-byte aligned.
 *   sa(m, kb) = sa[(m >> a_shift) * sa_row + kb * sa_col]
 *   sb(n, kb) = sb[(n >> b_shift) * sb_row + kb * sb_col]
 *      shift 0: per row (1x128 tiles, or channel with *_col = 0);
 *      shift 7: per 128-row block (128x128 blocks);  row = col = 0: tensor.
 *   bias optional [N] (bias_dtype); y [M, N] with row stride ldy, y_dtype.
 *   nan_a / nan_b optional int32 [M] / [N] row flags from the quantizers:
 *      a flagged row of A (or of B) makes its output row (column) NaN, as
 *      the NaN would in the reference's fp32 GEMM.
 */
int ntlb_gemm_blockscaled(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row, int64_t sa_col,
                          int a_shift, const uint8_t* b, int64_t ldb, const float* sb, int64_t sb_row,
                          int64_t sb_col, int b_shift, int64_t M, int64_t N, int64_t Kp, const void* bias,
                          int bias_dtype, void* y, int y_dtype, int64_t ldy, const int32_t* nan_a,
                          const int32_t* nan_b, void* stream);

/*
 * ntlb_gemm_blockscaled with a workspace for the tail of the tiling (the
 * same product as te_backend.py:253-259).  256x256 output tiles run one per
 * compute unit; when the tiles past the last whole wave would leave at least
 * half the compute units idle, each of them is split into 2..8 K ranges whose
 * fp32 partials meet in the workspace and are summed in a fixed order by the
 * last range to finish (deterministic; no waiting on other workgroups).
 *   workspace  256-byte aligned device memory of ws_bytes, ZEROED once before
 *              its first use; every call leaves it ready for the next.  Calls
 *              that may run concurrently need separate workspaces.
 *   ws_bytes   at least ntlb_gemm_workspace_bytes(M, N, Kp), else (or with a
 *              null workspace) the call runs unsplit like ntlb_gemm_blockscaled.
 */
int ntlb_gemm_blockscaled_ws(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                             int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, const float* sb,
                             int64_t sb_row, int64_t sb_col, int b_shift, int64_t M, int64_t N, int64_t Kp,
                             const void* bias, int bias_dtype, void* y, int y_dtype, int64_t ldy,
                             const int32_t* nan_a, const int32_t* nan_b, void* workspace, int64_t ws_bytes,
                             void* stream);

/* Workspace bytes ntlb_gemm_blockscaled_ws uses for this shape on the current
 * device (0: the shape runs unsplit). */
int64_t ntlb_gemm_workspace_bytes(int64_t M, int64_t N, int64_t Kp);

/*
 * GEMMs over the operands the reference actually multiplies.  The emulated
 * backend casts every dequantized operand back to the input dtype
 * (`.to(dtype=x.dtype)`, te_backend.py:173, :185, :193, :202) before its fp32
 * F.linear (te_backend.py:253-259), so for bf16 inputs each operand is
 * bf16(q * s).  These entry points decode codes + scales to exactly those
 * values inside the GEMM's tile prologue (no dequantized tensor is written)
 * and multiply them on bf16 MFMA (fp32 MFMA for op_dtype NTLB_F32) with fp32
 * accumulation: products of bf16 values are exact in fp32, so the result is
 * the reference's fp32 GEMM up to the order of the fp32 additions.
 *   op_dtype  the dtype the reference rounds the dequantized operands to:
 *             NTLB_BF16 or NTLB_F32 (NTLB_EUNSUPPORTED otherwise)
 * Codes, scales and their indexing follow ntlb_gemm_blockscaled: scale of
 * element (row, k) = s[(row >> shift) * s_row + (k >> 7) * s_col].  Int-grid
 * code -128 (a NaN element) decodes to NaN.
 */

/* Forward of EmulatedLowBitBackend.linear (te_backend.py:229-260) with the
 * reference's operand rounding: Y = bf16(dq(A)) . bf16(dq(B))^T + bias, cast
 * to y_dtype.  Same arguments as ntlb_gemm_blockscaled without the NaN flags
 * (NaN codes decode to NaN and propagate through the products). */
int ntlb_gemm_dq_forward(int op_dtype, int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                         int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, const float* sb, int64_t sb_row,
                         int64_t sb_col, int b_shift, int64_t M, int64_t N, int64_t Kp, const void* bias,
                         int bias_dtype, void* y, int y_dtype, int64_t ldy, void* stream);

/* Input gradient of the straight-through estimator (autograd of
 * te_backend.py:250-259): dX[M, K] = dY[M, N] . bf16(dq(W))[N, K], fp32
 * accumulation, cast to dx_dtype.  dY is the unquantized bf16 gradient, row
 * stride lddy >= N rounded up to 64 with ZERO pad columns [N, that), 16-byte
 * rows; W the forward's codes [N, ldw] with its scales (w_shift, sw_row,
 * sw_col as ntlb_gemm_blockscaled's B operand), read in place as the
 * transposed operand.  op_dtype NTLB_BF16 only; N > 0 (M or K == 0: no-op). */
int ntlb_gemm_ste_dgrad(int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N, int grid, const uint8_t* w,
                        int64_t ldw, const float* sw, int64_t sw_row, int64_t sw_col, int w_shift, int64_t K, void* dx,
                        int dx_dtype, int64_t lddx, void* stream);

/* ntlb_gemm_ste_dgrad with a split-K workspace (same interface as
 * ntlb_gemm_blockscaled_ws's): the output tiles past the last whole wave of
 * workgroups run as K ranges whose fp32 partials are summed in range order.
 * The workspace is 256-byte aligned, zeroed before its first use and left
 * zeroed; ws_bytes >= ntlb_gemm_dq_workspace_bytes(op_dtype, M, K, N), else
 * (or with NULL) the call runs unsplit.  Same autograd of te_backend.py:250-259. */
int ntlb_gemm_ste_dgrad_ws(int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N, int grid,
                           const uint8_t* w, int64_t ldw, const float* sw, int64_t sw_row, int64_t sw_col, int w_shift,
                           int64_t K, void* dx, int dx_dtype, int64_t lddx, void* workspace, int64_t ws_bytes,
                           void* stream);

/* Split-K workspace bytes of a dequantized-operand GEMM with an [M, N] output
 * and contraction Kc (0: the shape runs unsplit).  No counterpart in the
 * reference: the workspace serves ntlb_gemm_ste_dgrad_ws. */
int64_t ntlb_gemm_dq_workspace_bytes(int op_dtype, int64_t M, int64_t N, int64_t Kc);

/* Weight gradient of the straight-through estimator: dW[N, K] =
 * dY[M, N]^T . bf16(dq(X))[M, K], fp32 accumulation over the M tokens, cast
 * to dw_dtype.  dY bf16 [M, N] (lddy % 8 == 0) and X's codes [M, ldx] are both
 * read in place as transposed operands; any M > 0 (the contraction is
 * zero-padded inside the kernel).  op_dtype NTLB_BF16 only. */
int ntlb_gemm_ste_wgrad(int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N, int grid, const uint8_t* x,
                        int64_t ldx, const float* sx, int64_t sx_row, int64_t sx_col, int x_shift, int64_t K, void* dw,
                        int dw_dtype, int64_t lddw, void* stream);

/* The same weight gradient, also writing the bias gradient db[N] = the sum
 * of dY over its M rows (F.linear's bias gradient under autograd of
 * te_backend.py:253-259), accumulated in fp32 from the dY tiles the kernel
 * stages anyway (no separate pass over dY) and stored in db_dtype; db NULL
 * skips it.  The sum runs in a fixed order (each 8-row group of a 64-row
 * step, the steps in order, then the eight waves' partials in order), so
 * repeated calls are bit-identical.  e4m3 codes only (grid NTLB_GRID_E4M3;
 * the int grid's decode leaves no registers for it: NTLB_EUNSUPPORTED). */
int ntlb_gemm_ste_wgrad_db(int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N, int grid,
                           const uint8_t* x, int64_t ldx, const float* sx, int64_t sx_row, int64_t sx_col, int x_shift,
                           int64_t K, void* dw, int dw_dtype, int64_t lddw, void* db, int db_dtype, void* stream);

/* The straight-through dgrad of every expert's Linear at once (the input
 * gradient of te_backend.py:250-259 for each expert of the single-rank loop,
 * moe.py:1062-1093 / LocalRoutedMoE :476-491): rows sorted by expert, expert e
 * owning rows [offsets[e], offsets[e+1]) (offsets int32 [n_experts + 1]);
 * dX[rows of e] = dY[rows of e] . bf16(dq(W_e)), W_e the codes [N, ldw] at
 * w + e*w_estride with 128x128 block (or tensor) scales at sw + e*sw_estride
 * (scale(n, k) = sw[(n >> w_shift)*sw_row + (k >> 7)*sw_col]).  dY bf16 [R, ldy]
 * with ld >= N rounded up to 64 and zero pad columns; dX [R, lddx] of
 * dx_dtype.  op_dtype NTLB_BF16 only. */
int ntlb_gemm_grouped_ste_dgrad(int op_dtype, const void* dy, int64_t lddy, int64_t R, int64_t N,
                                const int32_t* offsets, int n_experts, int grid, const uint8_t* w, int64_t ldw,
                                int64_t w_estride, const float* sw, int64_t sw_row, int64_t sw_col, int w_shift,
                                int64_t sw_estride, int64_t K, void* dx, int dx_dtype, int64_t lddx, void* stream);

/* The input gradient of every expert's gate and up Linears (moe.py:190-193)
 * as autograd forms it: dX = bf16(dX_gate) + bf16(dX_up), added in bf16, with
 * dX_gate = d_gate . bf16(dq(W_gate)) and dX_up = d_up . bf16(dq(W_up)) over
 * the interleaved gate/up layout: d_gate_up bf16 [R, 2I] and the codes
 * [2I, ldw] of each expert (at w + e*w_estride, 128x128 block scales at sw +
 * e*sw_estride) hold 128-wide blocks alternating gate block t and up block t.
 * Rows sorted by expert (offsets int32 [n_experts + 1]); dX bf16 [R, lddx]. */
int ntlb_gemm_grouped_ste_dgrad_gate_up(int op_dtype, const void* dgu, int64_t lddgu, int64_t R, int64_t I,
                                        const int32_t* offsets, int n_experts, int grid, const uint8_t* w,
                                        int64_t ldw, int64_t w_estride, const float* sw, int64_t sw_row,
                                        int64_t sw_col, int64_t sw_estride, int64_t K, void* dx, int64_t lddx,
                                        void* stream);

/* The straight-through wgrad of every expert's Linear at once: dW_e[N, K] =
 * dY[rows of e]^T . bf16(dq(X[rows of e])) with the contraction over expert
 * e's rows only, for every expert (an expert without rows gets zeros); dW_e at
 * dw + e*dw_estride BYTES, row stride lddw.  X's codes [R, ldx] carry per-row
 * 1x128 scales in the tile-major layout (sx_row 1, sx_col a multiple of 4,
 * x_shift 0).  op_dtype NTLB_BF16 only. */
int ntlb_gemm_grouped_ste_wgrad(int op_dtype, const void* dy, int64_t lddy, int64_t R, int64_t N,
                                const int32_t* offsets, int n_experts, int grid, const uint8_t* x, int64_t ldx,
                                const float* sx, int64_t sx_row, int64_t sx_col, int x_shift, int64_t K, void* dw,
                                int dw_dtype, int64_t lddw, int64_t dw_estride, void* stream);

/*
 * The three grouped backward GEMMs of the expert loop over dense bf16
 * operands instead of codes: under stochastic rounding the reference's
 * straight-through operands t + (t_dq - t) (te_backend.py:250-251, formed by
 * ntlb_ste_value) differ from bf16(q * s), so the expert loop's backward
 * multiplies them directly, as each expert Linear's autograd does
 * (moe.py:1062-1093).
 *   ntlb_gemm_grouped_dgrad_dense: dX rows of expert e = dY rows [R, N] (ld
 *     >= N rounded up to 64, zero pad columns) . w_e, w [E][N][ldw] bf16 at
 *     w + e * w_estride (elements), dX [R, K].
 *   ntlb_gemm_grouped_dgrad_dense_gate_up: the interleaved gate / up form of
 *     ntlb_gemm_grouped_ste_dgrad_gate_up over w [E][2I][ldw].
 *   ntlb_gemm_grouped_wgrad_dense: dW_e [N, K] = dY rows^T . X rows over the
 *     expert's rows, X bf16 [R, ldx]; dW at dw + e * dw_estride bytes (zero
 *     for an expert without rows).
 * ld % 4 == 0 and 16-byte alignment for the operands read transposed.
 */
int ntlb_gemm_grouped_dgrad_dense(int op_dtype, const void* dy, int64_t lddy, int64_t R, int64_t N,
                                  const int32_t* offsets, int n_experts, const void* w, int64_t ldw, int64_t w_estride,
                                  int64_t K, void* dx, int dx_dtype, int64_t lddx, void* stream);
int ntlb_gemm_grouped_dgrad_dense_gate_up(int op_dtype, const void* dgu, int64_t lddgu, int64_t R, int64_t I,
                                          const int32_t* offsets, int n_experts, const void* w, int64_t ldw,
                                          int64_t w_estride, int64_t K, void* dx, int64_t lddx, void* stream);
int ntlb_gemm_grouped_wgrad_dense(int op_dtype, const void* dy, int64_t lddy, int64_t R, int64_t N,
                                  const int32_t* offsets, int n_experts, const void* x, int64_t ldx, int64_t K,
                                  void* dw, int dw_dtype, int64_t lddw, int64_t dw_estride, void* stream);

/* Y[M, N] = A[M, K] . op(B) + bias over bf16 or fp32 matrices (op_dtype), for
 * the dequantized tensors of granularities whose scales change along the
 * contraction element by element (the activation "channel" granularity of
 * te_backend.py:175-185).  A row-major [M, K] (a_trans must be 0); B [N, K]
 * (b_trans 0) or [K, N] (b_trans 1).  K a multiple of 64 (bf16) / 32 (fp32),
 * rows 16-byte aligned. */
int ntlb_gemm_dense(int op_dtype, const void* a, int64_t lda, int a_trans, const void* b, int64_t ldb, int b_trans,
                    int64_t M, int64_t N, int64_t K, const void* bias, int bias_dtype, void* y, int y_dtype,
                    int64_t ldy, void* stream);

/* Y[M, N] = A^T . B with A stored [K, M] and B stored [K, N] (the weight
 * gradient dY^T . X_dq over dequantized tensors); any K. */
int ntlb_gemm_dense_tn(int op_dtype, const void* a, int64_t lda, const void* b, int64_t ldb, int64_t M, int64_t N,
                       int64_t K, void* y, int y_dtype, int64_t ldy, void* stream);

/* Bias gradient of F.linear (te_backend.py:253-259 under autograd):
 * out[n] = sum over m of x[m, n] in fp32, cast to out_dtype.  Deterministic:
 * fp32 partials per 256-row chunk in `workspace` (fp32, at least
 * ntlb_colsum_workspace_bytes(M, N) bytes), added in chunk order. */
int ntlb_colsum(const void* x, int x_dtype, int64_t M, int64_t N, int64_t ldx, float* workspace, int64_t ws_bytes,
                void* out, int out_dtype, void* stream);

/* Workspace bytes of ntlb_colsum. */
int64_t ntlb_colsum_workspace_bytes(int64_t M, int64_t N);

/* The straight-through operand of EmulatedLowBitBackend.linear
 * (te_backend.py:250-251: `input + (input_dq - input).detach()`, and the same
 * for the weight): out[i] = t[i] + (t_dq[i] - t[i]) over n contiguous
 * elements of `dtype`, each operation in fp32 rounded to the dtype as torch
 * rounds it.  Equal to t_dq under round to nearest; under stochastic
 * rounding it is the operand the reference multiplies. */
int ntlb_ste_value(int dtype, const void* t, const void* t_dq, void* out, int64_t n, void* stream);

/*
 * Grouped (per-expert) blockwise-scaled GEMM over a token-offset table.
 * Replaces the per-expert loop of _run_local_experts (moe.py:888-962) /
 * _forward_single_rank (moe.py:1062-1097) in which every expert's Linear runs
 * the emulated backend on its selected rows.  Rows of A are sorted by expert:
 * expert e owns rows [offsets[e], offsets[e+1]) (int32 [E+1], device memory,
 * offsets[E] == M_total) and multiplies weight codes b + e*b_estride
 * ([N, Kp] each, row stride ldb) with scales sb + e*sb_estride.  Scale
 * indexing as ntlb_gemm_blockscaled, with A rows indexed globally.  Output
 * y [M_total, N].  nan_b, when given, is [E, N].  No host synchronization.
 */
int ntlb_gemm_grouped_blockscaled(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                                  int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, int64_t b_estride,
                                  const float* sb, int64_t sb_row, int64_t sb_col, int b_shift, int64_t sb_estride,
                                  const int32_t* offsets, int n_experts, int64_t M_total, int64_t N, int64_t Kp,
                                  void* y, int y_dtype, int64_t ldy, const int32_t* nan_a, const int32_t* nan_b,
                                  void* stream);

/*
 * Gate and up projections of the SwiGLU expert MLP in one blockscaled GEMM,
 * with h = silu(gate) * up and its 1x128 quantization in the epilogue.
 * Replaces F.silu(self.gate_proj(x)) * self.up_proj(x) (moe.py:190-193) and
 * the 1x128 quantization the down projection's backend applies to it
 * (te_backend.py:82-110), so h never makes an HBM round trip in fp32 or bf16.
 *   b, sb   interleaved weight: 128-row blocks gate block t, up block t, ...,
 *           N = 2*I rows (I a multiple of 128), 128x128 block scales
 *           (sb_row, sb_col) of the interleaved rows
 *   h       optional bf16 [M, I] (row stride ldh): bf16(silu(g) * u) with
 *           g, u the bf16-rounded projections and silu(x) = x / (1 + exp(-x))
 *           in fp32 rounded to bf16, as F.silu on a bf16 tensor
 *   hc, hs  h codes [M, ldhc] and scales hs[row*hs_row + tile*hs_col] with
 *           the grid, qmax, rounding, scale rule and SR (seed, offset) of
 *           ntlb_quant_tile_1x128 applied to h (SR keyed by row*I + column)
 *   h_nan   optional per-row NaN flags of h
 * nan_a / nan_b flag NaN rows of A and of the interleaved B as in
 * ntlb_gemm_blockscaled.
 */
int ntlb_gemm_swiglu_quant(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row, int64_t sa_col,
                           int a_shift, const uint8_t* b, int64_t ldb, const float* sb, int64_t sb_row,
                           int64_t sb_col, int64_t M, int64_t N, int64_t Kp, const int32_t* nan_a,
                           const int32_t* nan_b, uint16_t* h, int64_t ldh, uint8_t* hc, int64_t ldhc, float* hs,
                           int64_t hs_row, int64_t hs_col, int32_t* h_nan, int qmax, int rounding, int scale_rule,
                           uint64_t seed, uint64_t offset, void* stream);

/*
 * Per-expert form of ntlb_gemm_swiglu_quant over rows sorted by expert (the
 * offsets table and expert strides of ntlb_gemm_grouped_blockscaled): the
 * gate/up half of the expert loop of moe.py:888-962 for all local experts.
 */
int ntlb_gemm_grouped_swiglu_quant(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                                   int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, int64_t b_estride,
                                   const float* sb, int64_t sb_row, int64_t sb_col, int64_t sb_estride,
                                   const int32_t* offsets, int n_experts, int64_t M_total, int64_t N, int64_t Kp,
                                   const int32_t* nan_a, const int32_t* nan_b, uint16_t* h, int64_t ldh, uint8_t* hc,
                                   int64_t ldhc, float* hs, int64_t hs_row, int64_t hs_col, int32_t* h_nan, int qmax,
                                   int rounding, int scale_rule, uint64_t seed, uint64_t offset, void* stream);

/* ntlb_gemm_grouped_swiglu_quant that also stores the projections' bf16
 * outputs (gate and up, each rounded to bf16 as the reference's Linears
 * return them) into gu [M_total, ldgu] in B's interleaved column order, for
 * the SwiGLU backward of ntlb_swiglu_backward (the activations autograd keeps
 * for F.silu(gate) * up, moe.py:190-193).  gu NULL stores nothing. */
int ntlb_gemm_grouped_swiglu_quant_gu(int grid, const uint8_t* a, int64_t lda, const float* sa, int64_t sa_row,
                                      int64_t sa_col, int a_shift, const uint8_t* b, int64_t ldb, int64_t b_estride,
                                      const float* sb, int64_t sb_row, int64_t sb_col, int64_t sb_estride,
                                      const int32_t* offsets, int n_experts, int64_t M_total, int64_t N, int64_t Kp,
                                      const int32_t* nan_a, const int32_t* nan_b, uint16_t* h, int64_t ldh,
                                      uint8_t* hc, int64_t ldhc, float* hs, int64_t hs_row, int64_t hs_col,
                                      int32_t* h_nan, int qmax, int rounding, int scale_rule, uint64_t seed,
                                      uint64_t offset, uint16_t* gu, int64_t ldgu, void* stream);

/*
 * NF4 refresh of a persistent weight (the flat tensor of n elements):
 * _quantize_nf4_persistent + _pack_nibbles (layers.py:130-139, :156-169).
 * One scale per run of `block` consecutive elements (K for per_channel on an
 * [N, K] weight, n for per_tensor, 64 for the 64-element recipe): scale = amax
 * if finite and > 0 else 1 (layers.py:86-101).  code = argmin over the NF4
 * codebook (layers.py:60-83) of |clamp(w/s, -1, 1) - cb|, first minimum wins.
 * packed [ceil(n/2)]: element 2i in the low nibble of byte i.  amax_ws is a
 * caller-zeroed uint32 workspace of ceil(n/block) words; scales [ceil(n/block)].
 */
int ntlb_nf4_quant(const void* w, int w_dtype, int64_t n, int64_t block, uint32_t* amax_ws, uint8_t* packed,
                   float* scales, void* stream);

/* cb[code] * scale cast to out_dtype: _unpack_nibbles + _dequantize_nf4_persistent
 * (layers.py:142-153, :172-184). */
int ntlb_nf4_dequant(const uint8_t* packed, const float* scales, int64_t n, int64_t block, void* out,
                     int out_dtype, void* stream);

/*
 * MXFP4 (OCP MX v1.0) refresh: 32-element blocks, e8m0 scale
 * X = 2^(floor(log2 amax) - 2) (exponent clamped to [-127, 127]; 0xFF when the
 * block holds a NaN or inf), e2m1 codes rounded to nearest even with
 * saturation, packed as NF4.  No reference function (benchmark config 5).
 */
int ntlb_mxfp4_quant(const void* w, int w_dtype, int64_t n, uint8_t* packed, uint8_t* scales, void* stream);
int ntlb_mxfp4_dequant(const uint8_t* packed, const uint8_t* scales, int64_t n, void* out, int out_dtype,
                       void* stream);

/*
 * Persistent FP8 (layers.py:104-127): scale = amax per block (K for
 * per_channel, n for per_tensor; finite and > 0 else 1), codes =
 * e4m3fn(clamp(w/s, -448, 448)); dequant = e4m3 value * scale cast to out_dtype.
 * amax_ws: caller-zeroed uint32 [ceil(n/block)].
 */
int ntlb_fp8_persistent_quant(const void* w, int w_dtype, int64_t n, int64_t block, uint32_t* amax_ws,
                              uint8_t* codes, float* scales, void* stream);
int ntlb_fp8_persistent_dequant(const uint8_t* codes, const float* scales, int64_t n, int64_t block, void* out,
                                int out_dtype, void* stream);

/*
 * One AdamW step of PrecisionAdamW.step (optimizer_runtime.py:68-116)
 * on fp32 main_param, exp_avg, exp_avg_sq [n] in place, with the gradient in
 * grad_dtype, optionally writing the parameter copy in param_dtype
 * (param.data.copy_(main_param_f.to(param.dtype))).  The float scalars are the
 * reference's Python-double values cast to float32: beta1, 1-beta1, beta2,
 * 1-beta2, eps, 1-lr*weight_decay, -lr/(1-beta1^step); inv_bc2_sqrt is
 * (float)(1.0 / (1-beta2^step)^0.5), the reciprocal taken in double, since
 * torch divides a tensor by a scalar as a multiplication by that reciprocal.
 * The operations are those of the reference's torch ops on the GPU:
 * add(alpha) = fma(alpha, b, a), addcmul = fma(value, t1*t2, self),
 * addcdiv = fma(value, t1/t2, self), sqrt correctly rounded.
 * refresh = 1 (NF4) or 2 (persistent FP8) also quantizes that parameter copy
 * as refresh_persistent_lowbit_params does (layers.py:353-407), scale = amax
 * of each block of `block` elements (a power of two in [8, 2048]), into the
 * packed nibbles or e4m3 bytes `codes` and fp32 `scales`; refresh = 0 skips it.
 * There is no reference function for the fusion (the reference refreshes in a
 * second pass after the step).
 */
int ntlb_adamw_step_refresh(float* main_param, const void* grad, int grad_dtype, float* exp_avg, float* exp_avg_sq,
                            void* param, int param_dtype, int64_t n, float beta1, float one_minus_beta1, float beta2,
                            float one_minus_beta2, float inv_bc2_sqrt, float eps, float decay, float neg_step_size,
                            int refresh, int64_t block, uint8_t* codes, float* scales, void* stream);

/*
 * Dequant-fused GEMMs: Y[M, N] = X[M, K] (bf16) . deq(W)[N, K]^T with fp32
 * accumulation on bf16 MFMA, W dequantized in the B-tile prologue exactly as
 * ntlb_nf4_dequant / ntlb_mxfp4_dequant would (bf16 of value * scale).  The
 * persistent-weight forward of _persistent_weight_ste + F.linear
 * (layers.py:409-436, :595-632) without materializing the bf16 weight.
 * K % 64 == 0; NF4 block divides K and is a multiple of 32, or 0 for a
 * single tensor scale; ldx % 8 == 0; y bf16 or fp32.
 */
int ntlb_gemm_nf4(const void* x, int64_t ldx, const uint8_t* w_packed, const float* w_scales, int64_t block,
                  int64_t M, int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy, void* stream);
int ntlb_gemm_mxfp4(const void* x, int64_t ldx, const uint8_t* w_packed, const uint8_t* w_scales, int64_t M,
                    int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy, void* stream);

/*
 * The same fused GEMM for the persistent FP8 weight: w_codes [N, K] e4m3
 * bytes (the float8_e4m3fn `_persistent_fp8_weight`), dequantized as
 * _dequantize_fp8_persistent (layers.py:120-127) would, bf16(value * scale),
 * then multiplied as F.linear(x, weight) in the persistent forward
 * (layers.py:409-436).  block = K for the per_channel scale [N] or 0 for
 * per_tensor; K % 64 == 0.
 */
int ntlb_gemm_fp8p(const void* x, int64_t ldx, const uint8_t* w_codes, const float* w_scales, int64_t block,
                   int64_t M, int64_t N, int64_t K, void* y, int y_dtype, int64_t ldy, void* stream);

/*
 * The dequant-fused GEMMs with a bias and a workspace: fmt NTLB_LOWBIT_NF4
 * (w packed nibbles, fp32 block scales, block as ntlb_gemm_nf4),
 * NTLB_LOWBIT_FP8P (w e4m3 bytes, block as ntlb_gemm_fp8p) or
 * NTLB_LOWBIT_MXFP4 (w packed e2m1, e8m0 scales; block ignored).  bias
 * optional [N] (bias_dtype), added in fp32 before the output rounding, as
 * F.linear(x, weight, bias) does in the persistent forward
 * (layers.py:595-632).  workspace (256-byte aligned, zeroed before its first
 * use; every call leaves it zeroed) of ws_bytes >=
 * ntlb_gemm_lowbit_workspace_bytes(M, N, K) enables the split-K tail: the
 * output tiles past the last whole wave of the grid are cut into 2-8 K ranges
 * when they would fill at most half the chip; NULL runs every tile whole.
 * Concurrent calls need separate workspaces.  No counterpart in the
 * reference beyond the fused forward (the bias and the workspace are this
 * interface's own).
 */
#define NTLB_LOWBIT_NF4 0
#define NTLB_LOWBIT_MXFP4 1
#define NTLB_LOWBIT_FP8P 2
int64_t ntlb_gemm_lowbit_workspace_bytes(int64_t M, int64_t N, int64_t K);
int ntlb_gemm_lowbit_ws(int fmt, const void* x, int64_t ldx, const uint8_t* w, const void* w_scales, int64_t block,
                        const void* bias, int bias_dtype, int64_t M, int64_t N, int64_t K, void* y, int y_dtype,
                        int64_t ldy, void* workspace, int64_t ws_bytes, void* stream);

/*
 * The input gradient of a persistent layer, dX[M, K] = dY[M, N] . deq(W),
 * with the weight decoded inside the GEMM instead of dequantized to a copy:
 * the straight-through backward of _persistent_weight_ste (layers.py:409-436,
 * dX = dY . w_q under autograd) for fmt NTLB_LOWBIT_NF4 (W's nibbles flat as
 * _quantize_nf4_persistent packs them, layers.py:130-169) or NTLB_LOWBIT_FP8P
 * (float8_e4m3fn codes [N, K], layers.py:104-127).  op_dtype NTLB_BF16: each
 * weight is codebook value (or e4m3 value) times scale in fp32, rounded to
 * bf16 as _dequantize_*_persistent(..., target_dtype=bf16) rounds it, on bf16
 * MFMA; NTLB_F32: the fp32 values on fp32 MFMA.  dY [M, lddy] in op_dtype with
 * lddy >= N rounded up to 64 (bf16) or 32 (fp32) and zero pad columns;
 * w_scales fp32, 16-byte aligned: one per weight row (block = K) or one for
 * all (block 0 or N*K); K % 4 == 0.  workspace as for ntlb_gemm_ste_dgrad_ws
 * (sized by ntlb_gemm_dq_workspace_bytes(op_dtype, M, K, N)); NULL runs
 * every tile whole.
 */
int ntlb_gemm_lowbit_dgrad_ws(int fmt, int op_dtype, const void* dy, int64_t lddy, int64_t M, int64_t N,
                              const uint8_t* w, const float* w_scales, int64_t block, int64_t K, void* dx,
                              int dx_dtype, int64_t lddx, void* workspace, int64_t ws_bytes, void* stream);

/*
 * The persistent forward Y[M, N] = x[M, K] . deq(W)^T (+ bias) where
 * ntlb_gemm_lowbit_ws does not apply: fp32 activations (op_dtype NTLB_F32,
 * fp32 weight values on fp32 MFMA) or bf16 activations with K % 64 != 0
 * (F.linear(x, _persistent_weight_ste(), bias), layers.py:409-436 and
 * :595-632, without the dequantized copy).  fmt NTLB_LOWBIT_NF4 or
 * NTLB_LOWBIT_FP8P as for ntlb_gemm_lowbit_dgrad_ws, one scale per weight row
 * (block = K) or one for all (0 or N*K), K % 4 == 0.  x [M, ldx] in op_dtype
 * with ldx >= K rounded up to 64 (bf16) or 32 (fp32) and zero pad columns;
 * the weight's codes past K (the next row's) are masked out of the
 * contraction.  bias (optional, any float dtype) is added in fp32 before the
 * output rounding.  workspace sized by ntlb_gemm_dq_workspace_bytes(op_dtype,
 * M, N, K); NULL runs every tile whole.
 */
int ntlb_gemm_lowbit_dq_forward_ws(int fmt, int op_dtype, const void* x, int64_t ldx, int64_t M, const uint8_t* w,
                                   const float* w_scales, int64_t block, int64_t N, int64_t K, const void* bias,
                                   int bias_dtype, void* y, int y_dtype, int64_t ldy, void* workspace,
                                   int64_t ws_bytes, void* stream);

/*
 * Expert-parallel dispatch wire format: one fixed-size record per routed
 * (token, slot) assignment, so that a single byte all-to-all replaces the
 * payload and four metadata all-to-alls of _dispatch_tokens
 * (moe.py:795-863).  Record of a row of H values:
 *   [0, S_OFF)      codes (1x128 tiles of the comm-quant, moe.py:808-814),
 *                   S_OFF = 128*ceil(H/128), zero codes past column H
 *   [S_OFF, ...)    ceil(H/128) fp32 tile scales
 *   [M_OFF, +32)    int32 token index, int32 top-k slot, int32 local expert,
 *                   int32 NaN flag, fp32 routing weight, 3 reserved int32,
 *                   M_OFF = S_OFF + round_up(4*ceil(H/128), 16)
 * ntlb_ep_record_bytes(H) = M_OFF + 32 (0 for H <= 0).
 */
int64_t ntlb_ep_record_bytes(int64_t H);

/*
 * Stable counting sort of n keys into buckets: bucket(i) = key(i) / divisor,
 * key(i) the int32 (key_dtype 0) or int64 (1) at keys + i*key_stride bytes.
 * pos[i] is i's place in bucket order (earlier keys first within a bucket),
 * inv[pos[i]] = i; counts[b] (int64) and offsets[b] (int32, b <= buckets,
 * exclusive prefix) are optional.  Sender: keys = topk_idx flattened,
 * divisor = experts_per_rank, buckets = ep_size gives the destination order
 * of _build_send_partitions (moe.py:670-717).  Receiver: keys = the records'
 * local-expert field (key_stride = record bytes), divisor 1, buckets = local
 * experts gives the grouping of _run_local_experts (moe.py:905-923) without
 * capacity drop.  ws: int32 workspace of ceil(n/256)*buckets elements.
 * buckets <= 4096.
 */
int ntlb_ep_partition(const void* keys, int key_dtype, int64_t key_stride, int64_t n, int64_t divisor, int buckets,
                      int32_t* pos, int32_t* inv, int64_t* counts, int32_t* offsets, int32_t* ws, int64_t ws_elems,
                      void* stream);

/*
 * Write the T*K send records: assignment a goes to record p = pos[a] (pos from
 * ntlb_ep_partition on topk_idx): token row a / K of tokens [T, H] (row
 * stride ldt) quantized per 1x128 tile with the quantizer arguments of
 * ntlb_quant_tile_1x128 (the SR element index is p*H + column, the row-major
 * index in the send buffer), slot a % K, local expert topk_idx[a] %
 * experts_per_rank, weight topk_w[a] (w_dtype) and the NaN flag.  Each token
 * row is read once and written to its K records.  topk_idx int32 (idx_dtype
 * 0) or int64 (1), [T, K] contiguous.  tokens bf16 or fp32, H % 8 == 0,
 * 16-byte aligned rows and records.
 */
int ntlb_ep_pack_records(const void* tokens, int x_dtype, int64_t T, int64_t H, int64_t ldt, const int32_t* pos,
                         const void* topk_idx, int idx_dtype, const void* topk_w, int w_dtype, int64_t K,
                         int64_t experts_per_rank, int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                         uint64_t offset, uint8_t* records, void* stream);

/*
 * ntlb_ep_pack_records with the reference's own comm-quant scales
 * (_comm_quant_dequant, moe.py:79-143, applied to the send buffer by
 * _dispatch_tokens, moe.py:805-814): one scale per gc-column group over all
 * rows, from the group amaxes of ntlb_amax_grouped on tokens [T, H] with gr =
 * T and the same gc (granularity tile_1x128 / block_128x128: gc = 128, one
 * strip per tile; tensor: gc = H).  gc % 128 == 0 or gc >= H.  Every record's
 * tile scales are its group's scale; codes as ntlb_quant_grouped writes them
 * (grid, qmax, rounding, scale_rule as there; the reference uses the int grid,
 * qmax 127 and NTLB_SCALE_BEFORE_DIVIDE).  amax_bits NULL gives
 * ntlb_ep_pack_records.
 */
int ntlb_ep_pack_records_grouped(const void* tokens, int x_dtype, int64_t T, int64_t H, int64_t ldt,
                                 const int32_t* pos, const void* topk_idx, int idx_dtype, const void* topk_w,
                                 int w_dtype, int64_t K, int64_t experts_per_rank, const uint32_t* amax_bits,
                                 int64_t gc, int grid, int qmax, int rounding, int scale_rule, uint64_t seed,
                                 uint64_t offset, uint8_t* records, void* stream);

/*
 * Expert side of the combine (moe.py:926-962, _combine_remote_outputs
 * :964-1038): row i of the expert outputs x [n, H] (row stride ldx) becomes
 * record pos[i] (pos from ntlb_ep_partition on the rows' source ranks, so
 * each destination's records keep expert order, as send_back_features_parts
 * does), with token_idx[i], slot_idx[i], the optional local expert and
 * weight, and the NaN flag.  Payload: per-row 1x128 tiles (amax_bits NULL,
 * the quantizer of ntlb_quant_tile_1x128) or group scales from
 * ntlb_amax_grouped on x with gr = n (as ntlb_ep_pack_records_grouped).  SR
 * element index p*H + column.  x bf16 or fp32, H % 8 == 0, 16-byte aligned
 * rows and records.
 */
int ntlb_ep_pack_return(const void* x, int x_dtype, int64_t n, int64_t H, int64_t ldx, const int32_t* pos,
                        const int32_t* token_idx, const int32_t* slot_idx, const int32_t* local_expert,
                        const float* weight, const uint32_t* amax_bits, int64_t gc, int grid, int qmax, int rounding,
                        int scale_rule, uint64_t seed, uint64_t offset, uint8_t* records, void* stream);

/*
 * Source side of the combine (moe.py:1021-1027): out[t] = the sum over token
 * t's returned records of topk_w[t, slot] * dequant(record), as the
 * reference's index_add_ into zeros forms it on the CPU: dequant = q * scale
 * rounded to out_dtype, each product rounded to out_dtype, the products
 * summed in fp32 in arrival order (for one token, ascending expert id
 * topk_idx[t, slot]) and the sum rounded to out_dtype once.  Assignments without a record (capacity drops)
 * add nothing; tokens without any stay zero.  n records of the grid's codes,
 * topk_idx int32 (idx_dtype 0) or int64 (1) and topk_w (w_dtype) [T, K]
 * contiguous, K <= 32, H % 8 == 0, out [T, ldo].  slot_map: int32 workspace
 * of T*K elements.
 */
int ntlb_ep_combine(const uint8_t* records, int64_t n, int64_t H, const void* topk_idx, int idx_dtype,
                    const void* topk_w, int w_dtype, int64_t T, int64_t K, int grid, void* out, int out_dtype,
                    int64_t ldo, int32_t* slot_map, void* stream);

/*
 * Receiver side: output row i < rows is record inv[i] of the n received
 * records (inv from ntlb_ep_partition on their local-expert field with rows =
 * n, or any selection the caller chooses, e.g. the rows kept by a capacity
 * drop, moe.py:919-923, with rows <= n or repeats): codes (128*ceil(H/128)
 * bytes with their zero padding, ldc at least that) to codes + i*ldc,
 * scales to scales[i*s_row + t*s_col], and the optional NaN flag, token
 * index, slot, routing weight and source rank (the s with recv_offsets[s] <=
 * inv[i] < recv_offsets[s+1]) -- the tensors of _DispatchedTokens
 * (moe.py:49-58) in expert order, with the payload kept as codes for the
 * grouped GEMM.  recv_offsets is HOST memory, int64 [ep_size + 1], the prefix
 * of the received counts from 0 to n (as recv_src_ranks is built from the
 * counts, moe.py:851-854), read during the call; needed only with src_rank;
 * ep_size <= 256.  n < 2^31.
 */
int ntlb_ep_unpack_records(const uint8_t* records, int64_t n, int64_t H, const int32_t* inv, int64_t rows,
                           const int64_t* recv_offsets, int ep_size, uint8_t* codes, int64_t ldc, float* scales,
                           int64_t s_row, int64_t s_col, int32_t* nan_rows, int32_t* token_idx, int32_t* slot_idx,
                           int32_t* src_rank, float* weight, void* stream);

/*
 * Value records: the payload is the row's values themselves, in the input
 * dtype, as the reference's comm-quant leaves them in its send buffers
 * (_comm_quant_dequant, moe.py:79-143, of send_tokens at :805-814 and of
 * send_back_features at :983-990): tensor + (dq - tensor) with dq = q * scale
 * rounded to the dtype.  This carries any column grouping of the scales,
 * including one per column (channel granularity, moe.py:112-121), which a
 * code record's tile scales cannot, and moves 2 (bf16) or 4 bytes per value,
 * as the reference's own exchange does.  Layout, in whole 128-byte lines so
 * that every payload starts on one:
 *   [0, P)          the H values, P = H * dtype size
 *   [P, R - 32)     zero padding
 *   [R - 32, R)     the metadata of a code record (token, slot, local expert,
 *                   0, fp32 weight, 3 reserved)
 * ntlb_ep_value_record_bytes(H, dtype) = R = round_up(P + 32, 128) (0 for H <=
 * 0 or a bad dtype).
 */
int64_t ntlb_ep_value_record_bytes(int64_t H, int dtype);

/*
 * ntlb_ep_pack_records_grouped with value records: assignment a -> record
 * pos[a], the token row a / K of tokens [T, H] quantized with one scale per
 * gc-column group over all rows (amax_bits from ntlb_amax_grouped on tokens
 * with gr = T and the same gc; gc = 1 channel, 128 tile_1x128 /
 * block_128x128, H tensor) and written as the straight-through value
 * ntlb_comm_quant_dequant forms for send-buffer row p (SR element index p*H
 * + column).  The values equal ntlb_comm_quant_dequant's on the send buffer
 * tokens[inv / K] bit for bit.  tokens bf16 or fp32, H % 8 == 0, 16-byte
 * aligned rows and records.
 */
int ntlb_ep_pack_values(const void* tokens, int x_dtype, int64_t T, int64_t H, int64_t ldt, const int32_t* pos,
                        const void* topk_idx, int idx_dtype, const void* topk_w, int w_dtype, int64_t K,
                        int64_t experts_per_rank, const uint32_t* amax_bits, int64_t gc, int grid, int qmax,
                        int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* records, void* stream);

/*
 * ntlb_ep_pack_return with value records: row i of x [n, H] -> record pos[i]
 * with token_idx[i], slot_idx[i], the optional local expert and weight, the
 * values quantized with the group scales of ntlb_amax_grouped on x (gr = n)
 * as in ntlb_ep_pack_values.
 */
int ntlb_ep_pack_return_values(const void* x, int x_dtype, int64_t n, int64_t H, int64_t ldx, const int32_t* pos,
                               const int32_t* token_idx, const int32_t* slot_idx, const int32_t* local_expert,
                               const float* weight, const uint32_t* amax_bits, int64_t gc, int grid, int qmax,
                               int rounding, int scale_rule, uint64_t seed, uint64_t offset, uint8_t* records,
                               void* stream);

/*
 * ntlb_ep_unpack_records for value records of val_dtype: row i < rows of
 * values [rows, ldv] (val_dtype) is the payload of record inv[i], with the
 * optional token index, slot, routing weight and source rank as there
 * (recv_offsets HOST memory, needed only with src_rank).  H % 8 == 0,
 * 16-byte aligned records and value rows.
 */
int ntlb_ep_unpack_values(const uint8_t* records, int64_t n, int64_t H, int val_dtype, const int32_t* inv,
                          int64_t rows, const int64_t* recv_offsets, int ep_size, void* values, int64_t ldv,
                          int32_t* token_idx, int32_t* slot_idx, int32_t* src_rank, float* weight, void* stream);

/*
 * ntlb_ep_combine for value records of val_dtype: each returned value
 * rounded to out_dtype (the reference's recv_back_features.to(tokens.dtype),
 * moe.py:998-999), times its routing weight rounded to out_dtype, the
 * products summed in fp32 in ascending expert id per token and the sum
 * rounded once; capacity drops add nothing.  Shapes as ntlb_ep_combine.
 */
int ntlb_ep_combine_values(const uint8_t* records, int64_t n, int64_t H, int val_dtype, const void* topk_idx,
                           int idx_dtype, const void* topk_w, int w_dtype, int64_t T, int64_t K, void* out,
                           int out_dtype, int64_t ldo, int32_t* slot_map, void* stream);
/*
 * Single-rank combine of the local experts' outputs (moe.py:1087-1088,
 * LocalRoutedMoE :489-490): out[t] starts at zero and, for token t's slots in
 * ascending expert id (the reference's expert loop order), takes
 * out[t] += y[pos[t*K + s]] * topk_w[t, s], the product in torch's promoted
 * dtype of (y, w) and the sum in the output dtype, each rounded on its own.
 * y [n, H] (row stride ldy) holds the expert outputs in the output dtype, rows
 * in expert order (pos from ntlb_ep_partition on topk_idx, the order of
 * ntlb_quant_tile_1x128_fanout); a negative pos entry (dropped) adds nothing,
 * entries at or past n are clamped to n - 1.  topk_idx int32 (idx_dtype 0)
 * or int64 (1) and topk_w (w_dtype) [T, K] contiguous, 1 <= K <= 32, out
 * [T, ldo].
 */
int ntlb_moe_combine_rows(const void* y, int64_t ldy, int64_t n, const int32_t* pos, const void* topk_idx,
                          int idx_dtype, const void* topk_w, int w_dtype, int64_t T, int64_t K, int64_t H, void* out,
                          int out_dtype, int64_t ldo, void* stream);
/*
 * Capacity keep of the single-rank expert loop (moe.py:1077-1081,
 * LocalRoutedMoE :482-486: keep_rel = torch.topk(sort_weights, k=capacity,
 * sorted=True).indices when an expert has more than `capacity` rows).  In:
 * the rows sorted by expert (inv [rows]: row -> assignment t*K + s, offsets
 * int32 [n_experts + 1], as ntlb_ep_partition gives them) and topk_w
 * (w_dtype, n_assign = T*K entries).  Out: the kept rows, each expert's
 * highest weight first (equal weights keep row order), as pos_out
 * [n_assign] (assignment -> kept row, -1 dropped), inv_out [rows] (kept row
 * -> assignment; -1 past the kept count), offsets_out
 * [n_experts + 1] and counts_out int64 [n_experts].  capacity <= 0 keeps every
 * row in its order.
 */
int ntlb_moe_capacity_keep(const int32_t* inv, const int32_t* offsets, int n_experts, int64_t rows, int64_t n_assign,
                           const void* topk_w, int w_dtype, int64_t capacity, int32_t* pos_out, int32_t* inv_out,
                           int32_t* offsets_out, int64_t* counts_out, void* stream);

/*
 * Backward of the single-rank combine `output[token_indices] += expert_out *
 * weights` (moe.py:1087-1088, :489-490): for token t's slot s with row r =
 * pos[t*K + s] >= 0, dy[r] = d_out[t] * topk_w[t, s] rounded to `dtype` (the
 * gradient of expert_out) and d_w[t, s] = sum over H of d_out[t] * y[r] in
 * fp32, stored in w_dtype (the gradient of the routing weight; when w_dtype
 * is dtype's 16-bit type, each product is rounded to it first, as torch's mul
 * backward forms them); a dropped slot
 * (r < 0) gets d_w = 0 and writes no row.  d_out [T, ldo], y [n, ldy] and dy
 * [n, lddy] share `dtype`; 1 <= K <= 8.
 */
int ntlb_moe_combine_backward(const void* d_out, int64_t ldo, const void* y, int64_t ldy, int dtype,
                              const int32_t* pos, const void* topk_w, int w_dtype, int64_t T, int64_t K, int64_t H,
                              void* dy, int64_t lddy, void* d_w, void* stream);

/*
 * Backward of gated = F.silu(gate) * up over bf16 tensors (ExpertMLP.forward,
 * moe.py:190-193): with s = bf16(silu(g)), d_up = bf16(d * s), d_s = bf16(d *
 * u) and d_gate = bf16(d_s * sig * (1 + g * (1 - sig))) (sig = 1 / (1 +
 * exp(-g)), torch's silu backward in fp32).  dh bf16 [R, I]; gu and dgu bf16
 * [R, 2I] in the interleaved column order of the fused gate/up GEMM (h column
 * j: gate column 256*(j/128) + j%128, up column that + 128); I % 128 == 0.
 */
int ntlb_swiglu_backward(const uint16_t* dh, int64_t lddh, const uint16_t* gu, int64_t ldgu, int64_t R, int64_t I,
                         uint16_t* dgu, int64_t lddgu, void* stream);

/*
 * The token gradient of the single-rank loop's gather `tokens[token_indices]`
 * (moe.py:1086, :488) under autograd: out[t] = the rows dx[pos[t*K + s]] of
 * token t's kept slots, summed in descending expert id with each add rounded
 * to `dtype` (the order in which autograd accumulates them: the later
 * experts' backward runs first); zero for a token with no kept slot.  dx and
 * out share `dtype`; topk_idx int32 (idx_dtype 0) or int64 (1) [T, K], 1 <= K
 * <= 8.
 */
int ntlb_moe_token_grad(const void* dx, int64_t lddx, int dtype, const int32_t* pos, const void* topk_idx,
                        int idx_dtype, int64_t T, int64_t K, int64_t H, void* out, int64_t ldo, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NTLOWBIT_H */
