/*
 * cormorant_hip.h -- C ABI of libcormo_hip.so: the five units of the fixed-point simulator
 * (VectorOP with its activation and softmax units, Matmul, Conv, Pooling, RowOps) as
 * gfx950 HIP kernels.
 *
 * Conventions (all entry points):
 *   - Tensors are DEVICE pointers to raw two's-complement lanes (value = raw * 2^-f):
 *     int16 unless stated, int32 / float32 where a row-ops kind says so.  The caller owns
 *     every buffer; outputs are written into preallocated memory.
 *   - Counts and strides are the reference unit's register values (elements unless a
 *     register is documented in bytes).
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Calls are
 *     asynchronous on that stream.  The library keeps per-device state that calls share:
 *     the unit tables, the row-ops parameter RAM and one grow-only workspace.  Calls that
 *     overlap on one device -- from two host threads, or queued on two streams whose work
 *     may run concurrently -- therefore race; order them (one stream, or events).
 *   - Workspace growth allocates (and keeps every outgrown buffer until the process ends,
 *     so graphs captured earlier stay valid); a call that would grow it while its stream
 *     captures a HIP graph fails with CM_EINVAL -- run that call once before the capture.
 *   - Return value: CM_OK (0) or a negative CM_E* status; cm_last_error() describes the
 *     last failure of the calling thread.  Nothing throws across the ABI.
 *
 * Each entry point cites the reference interface it replaces (paths relative to the
 * reference checkout).
 */
#ifndef CORMORANT_HIP_H
#define CORMORANT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CM_OK 0
#define CM_EINVAL (-1)   /* a register value outside the unit's contract */
#define CM_EALIGN (-2)   /* a pointer or stride breaks the 16-byte word contract */
#define CM_EHIP (-3)     /* a HIP runtime call failed */
#define CM_ENOMEM (-4)   /* workspace allocation failed */

/* Version of this ABI (major * 100 + minor). */
int cm_abi_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char* cm_last_error(void);

/* Prepare the current device: builds the activation tables (glibc double formulas,
 * vectorop_act.py:60-114), the softmax exponential table (vectorop_smx.py:29-34) and the
 * row-ops table image (rowops_spec.py:605-616) and uploads them.  Every entry point calls
 * it on first use of a device; calling it first keeps that work out of timed regions. */
int cm_init(void);

/* Host-side copies of the tables cm_init builds (no device work): the full 65 536-entry
 * activation table of act 4 (SiLU), 5 (GELU erf) or 6 (GELU tanh), ascending raw input
 * (vectorop_act.kernel_table, vectorop_act.py:107-114); and the 64 KiB row-ops table image
 * (rowops_spec.table_image, rowops_spec.py:605-616). */
int cm_host_act_table(int act, int16_t* out65536);
int cm_host_rowops_table_image(uint8_t* out65536);

/* The current device's unit tables from the caller (the role of cm_act_table_init /
 * cm_rowops_tables_init in the boundary the reference's simulator mirrors; cm_init builds
 * both from the RTL ROM text and rowops_spec): `tables` = host int16 [3][65536], f(x) at
 * [x + 32768] for act 4 (SiLU), 5 (GELU), 6 (GELU-tanh), each of the form max(x, 0) - d[|x|]
 * with d a byte table of at most 4096 entries (CM_EINVAL otherwise, the tables unchanged);
 * `img64k` = the 64 KiB row-ops table image (ROWOPS_RTL_KERNEL.md section 1.4, what a TLOAD
 * job loads).  Blocking copies: call with no unit work of this library in flight. */
int cm_act_table_init(const int16_t* tables);
int cm_rowops_tables_init(const void* img64k);

/* Kernel timing (the role of the board runtime's per-call profiler,
 * inference-scheduler/runtime/inference_prof.c): while enabled, every kernel launch of the
 * library records a HIP event pair on its stream; on a stream under graph capture the pair
 * is two event-record nodes of the graph, re-recorded by each replay (read the records after
 * a replay).  cm_timing_read waits for the recorded
 * launches of `kernel` (a name such as "gemm_planes_kernel") and returns their summed
 * duration and count; cm_timing_reset drops every record. */
int cm_timing_enable(int on);
int cm_timing_read(const char* kernel, double* total_ms, uint64_t* launches);
int cm_timing_reset(void);
/* Record only the launches of `kernel` (NULL or "": every kernel), so that timing one
 * kernel inside a loop adds two events per launch of it and none elsewhere.  The events
 * skip the system-scope fence, so they neither flush caches nor slow the launches after. */
int cm_timing_select(const char* kernel);
/* The recorded launches of `kernel` one by one, in launch order: their durations (ms) into
 * ms[0 .. min(cap, count)), the count into *launches.  Waits for them as cm_timing_read. */
int cm_timing_read_each(const char* kernel, double* ms, uint64_t cap, uint64_t* launches);

/* ---------------------------------------------------------------- VectorOP
 * Replaces VectorOPKernel (kernels/vectorop_rtl/model/include/VectorOP.h:319-333) and the
 * simulator's VectorOP branch (inference-scheduler/src/codegen/_simulate.py:721-765), the
 * activation unit (vectorop_act.py:60-114) and the softmax unit
 * (vectorop_smx.py:37-79, smx_nodes.py:121-338):
 *   op 0..9: c[o*(a_inc+b_inc) + i] = act(op(a[o*a_inc + i], b[o*b_inc + i])),
 *            o < outer, i < size; b is not read for the unary ops (op >= 4);
 *   op 10:   softmax rows: row o at a + o*a_inc -> c + o*b_inc, o < outer;
 *   op 11:   softmax columns: s[size keys][outer queries] (row stride a_inc) ->
 *            P[q][size] at c + q*b_inc for q < (outer & ~15).
 * Every run is written as whole 8-lane (16-byte) words, the lanes past `size` 0, so `c`
 * must cover them; a, b, c 16-byte aligned; a_inc and b_inc multiples of 8 (or 0) for
 * ops 0..9 (the unit's alignment contract, VectorOP.h:222-236).  Softmax rows take
 * size <= 65535.  DIV follows the simulator: trunc(a*256/b) saturated, b == 0 gives
 * +32767 (a > 0), -32768 (a < 0), 0 (a == 0). */
int cm_vectorop(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size, uint32_t op,
                uint32_t outer, uint32_t a_inc, uint32_t b_inc, uint32_t act, uint32_t alpha,
                uint32_t smx_cm, uint32_t smx_cfg, uint32_t smx_mask, void* stream);

/* cm_vectorop for ops 0..9 over `outer` runs of `size` (a multiple of 64, up to 32768) whose
 * outputs are contiguous rows (a_inc + b_inc == size), also writing the output's byte planes
 * for a following cm_matmul_aplanes with A = c (n = outer, k = size): `planes` holds
 * cm_matmul_a_planes_bytes(outer, size, ceil(size / 1024)) bytes, 256-byte aligned.  c is what
 * cm_vectorop writes; c may be NULL when only the matmul reads the output (the planes alone
 * are written).  No counterpart in the reference: the operand split of this build's matmul,
 * done by the VectorOP call that produces the operand. */
int cm_vectorop_planes(const int16_t* a, const int16_t* b, int16_t* c, uint32_t size, uint32_t op, uint32_t outer,
                       uint32_t a_inc, uint32_t b_inc, uint32_t act, uint32_t alpha, void* planes, void* stream);

/* The softmax unit over a batch of matrices (the per-head VectorOPKernel softmax calls of
 * SoftmaxVopNode / VitAttnSoftmaxVopNode / LlmAttnSoftmaxVopNode, smx_nodes.py:121-338, in
 * one launch): matrix i reads a + i * a_bs and writes c + i * c_bs (elements), each exactly
 * cm_vectorop(a_i, NULL, c_i, size, op, outer, a_inc, c_inc, 0, 0, smx_cm, smx_cfg,
 * smx_mask).  op 10: rows [outer][size]; op 11: keys-major s[size][outer] -> P[outer][size],
 * size <= 1024. */
int cm_softmax(const int16_t* a, int16_t* c, uint32_t size, uint32_t op, uint32_t outer,
               uint32_t a_inc, uint32_t c_inc, uint32_t smx_cm, uint32_t smx_cfg, uint32_t smx_mask,
               uint32_t batch, uint64_t a_bs, uint64_t c_bs, void* stream);

/* ---------------------------------------------------------------- Matmul
 * Replaces MatmulKernel (kernels/matmul_rtl/model/include/MatmulKernel.h:228-242) and the
 * simulator's MatMul branches (_simulate.py:620-633 Q8.8, :814-835 power-of-two):
 *   C[bt][i][j] = sat16(floor(acc / 2^8)), acc = sum_kk A[bt][i][kk] * B[bt][kk][j]
 * with n rows of A, k inner, m columns of B, `batch` slices a_bs / b_bs / c_bs elements
 * apart (0 = broadcast).  acc is exact (wrap32 = 0, the simulator's Q8.8 path) or wrapped
 * to int32 first (wrap32 = 1, the power-of-two path).  B image: b_packed = 0 row-major
 * [k][m]; 1 the tile-major packed layout ((j/32)*k + kk)*32 + j%32 (MatmulKernel.h:91-113);
 * gemv_kw in {1,2,4,8} the kernel-width image (MatmulKernel.h:115-156); b_packed = 2 (this
 * build's addition, no MatmulKernel image) the transposed image [m][k], B[kk][j] = b[j*k + kk]:
 * q.K^T straight from the K rows of an attention cache.  C is row-major [n][m].  Limits:
 * 1 <= k <= 32768 (the unit takes 4096).  MatmulKernel's last register, a_to_b (GEMV mode:
 * address of b minus address of a, MatmulKernel.h:141-143, 216, 241), has no argument here:
 * it exists because an m_axi port knows only its own base address, and a device pointer to B
 * is passed directly instead; the GEMV image is read through b with gemv_kw as above. */
int cm_matmul(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
              uint32_t m, uint32_t batch, int64_t a_bs, int64_t b_bs, int64_t c_bs,
              uint32_t b_packed, uint32_t gemv_kw, uint32_t wrap32, void* stream);

/* cm_matmul without any allocation (no counterpart in the reference: for callers that cannot
 * allocate device memory, e.g. code under HIP graph capture or a serving loop that forbids
 * it).  Same arguments and results as cm_matmul; the operand planes, line sums and split-k
 * partials live in a device array of CM_NOALLOC_MAX_BYTES that the library's code object
 * holds on each device, and a call that needs more returns CM_EINVAL.  cm_init must have run
 * on the current device (CM_EINVAL otherwise: set-up allocates the unit tables).  Every call
 * on a device shares that device's array, so calls that overlap on one device race; no byte
 * of it needs to start at zero (each call writes what it reads). */
#define CM_NOALLOC_MAX_BYTES ((size_t)64 << 20)
int cm_matmul_noalloc(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k,
                      uint32_t m, uint32_t batch, int64_t a_bs, int64_t b_bs, int64_t c_bs,
                      uint32_t b_packed, uint32_t gemv_kw, uint32_t wrap32, void* stream);

/* Up to 4 int32-wrap products of the same A rows (n <= 32, the decode step's q / k / v or gate /
 * up projections) in one launch (no counterpart in the reference's units: each product is
 * cm_matmul(a, b[i], c[i], n, k, m[i], 1, 0, 0, n m[i], b_packed, 0, 1) of MatmulKernel.h:228-242,
 * the same results): C_i = sat16(wrap32(A . B_i) >> 8).  b_packed 0 / 1 / 2 as cm_matmul; m[i]
 * even (a multiple of 32 packed), k even (a multiple of 8 and 16-byte aligned B transposed). */
int cm_matmul_skinny_multi(const int16_t* a, uint32_t n, uint32_t k, uint32_t count, const int16_t* const* b,
                           int16_t* const* c, const uint32_t* m, uint32_t b_packed, void* stream);

/* The products of cm_matmul_skinny_multi (n <= 16 rows, k a multiple of 8, a 16-byte aligned)
 * against weights already split by cm_matmul_split_b (b_slices 1, the same k and m[i]): C_i =
 * sat16(wrap32(A . B_i) >> 8), C_i row-major [n][m[i]].  No counterpart in the reference's
 * units (each product is the MatmulKernel call of cm_matmul, MatmulKernel.h:228-242): one
 * launch, no workspace, for the decode step's linears. */
int cm_matmul_skinny_planes(const int16_t* a, uint32_t n, uint32_t k, uint32_t count, const void* const* b_planes,
                            int16_t* const* c, const uint32_t* m, void* stream);

/* cm_matmul_skinny_planes by the saturating Q8.8 rule (MatmulKernel's wrap32 = 0): C_i =
 * sat16(floor(A . B_i / 2^8)) with the sum exact, as cm_matmul with wrap32 = 0 writes it (the
 * same operands, n <= 16, k a multiple of 8).  No counterpart in the reference's units (each
 * product is the MatmulKernel call of cm_matmul, MatmulKernel.h:228-242): one launch, no
 * workspace, for few-row products of a constant weight (a classifier at a small batch). */
int cm_matmul_skinny_planes_sat(const int16_t* a, uint32_t n, uint32_t k, uint32_t count,
                                const void* const* b_planes, int16_t* const* c, const uint32_t* m, void* stream);

/* One product of cm_matmul_skinny_planes followed, in the same launch, by a row-ops COPY /
 * ADDX job on its output (the decode step's residual add): C = sat16(wrap32(A . B) >> 8) as
 * there, then out[r][j] = the job of op word `op` (A kind int16 / int32, B the int16 C, output
 * kind int16 / int32, F_P_BCAST / F_RELU / F_SCALE) over x[r][j] and C[r][j] with the 16-byte
 * parameter block `params` and bq_sh -- the cm_rowops job (x, c, out, params, op, n = m, c1 = n)
 * of ROWOPS_RTL_KERNEL.md section 1 on whole rows (x and out row-major [n][m]).  No
 * counterpart in the reference's units; the results equal those two calls. */
int cm_matmul_skinny_planes_addx(const int16_t* a, uint32_t n, uint32_t k, const void* b_planes, int16_t* c,
                                 uint32_t m, const void* x, const void* params, uint32_t op, uint32_t bq_sh,
                                 void* out, void* stream);

/* Two products of cm_matmul_skinny_planes over the same A -- a gate and an up weight of m
 * columns each -- and the row-ops MULACT job over their outputs in one launch (the decode
 * step's SiLU gate): c_gate and c_up as cm_matmul_skinny_planes writes them, then out[r][j] =
 * the job of op word `op` (int16 A, B and output, B enabled, F_P_BCAST) over c_gate[r][j] and
 * c_up[r][j] with the 16-byte parameter block `params` -- the cm_rowops job (c_gate, c_up, out,
 * params, op, n = m, c1 = n) of ROWOPS_RTL_KERNEL.md section 1 on whole rows (m <= 4096).  The
 * device's row-ops parameter RAM is left as it was.  No counterpart in the reference's units; the results
 * equal those calls. */
int cm_matmul_skinny_planes_mulact(const int16_t* a, uint32_t n, uint32_t k, const void* b_gate, const void* b_up,
                                   int16_t* c_gate, int16_t* c_up, uint32_t m, const void* params, uint32_t op,
                                   int16_t* out, void* stream);

/* cm_matmul over strided operands (no counterpart in the reference's units: the per-head
 * operands that VitAttnPrep / LlmAttnMerge would copy out and back, read and written in place):
 * slice bt of `batch` starts at (bt / inner) x_bs + (bt % inner) x_bs2 elements of each
 * operand (bt x_bs with inner 1); A[i][kk] = a[.. + i lda + kk]; B[kk][j] = b[.. + kk ldb + j],
 * or b[.. + j ldb + kk] with b_trans; C[i][j] at c[.. + i ldc + j]; the arithmetic of
 * cm_matmul.  16-byte aligned operands and strides (elements multiples of 8), k % 8 == 0, and
 * m % 8 == 0 without b_trans. */
int cm_matmul_strided(const int16_t* a, const int16_t* b, int16_t* c, uint32_t n, uint32_t k, uint32_t m,
                      uint32_t batch, uint32_t inner, uint64_t lda, uint64_t a_bs, uint64_t a_bs2, uint64_t ldb,
                      uint64_t b_bs, uint64_t b_bs2, uint32_t b_trans, uint64_t ldc, uint64_t c_bs, uint64_t c_bs2,
                      uint32_t wrap32, void* stream);

/* A constant B (a weight read by many calls) split once: cm_matmul_split_b writes B's byte
 * planes and line sums -- what every cm_matmul call otherwise derives from b on the fly --
 * into `planes` (cm_matmul_b_planes_bytes(k, m, b_slices) bytes, 256-byte aligned), from the
 * same b image, layout and b_bs as cm_matmul; cm_matmul_planes then computes exactly
 * cm_matmul(a, b, c, n, k, m, batch, a_bs, b_slices > 1 ? b_bs : 0, c_bs, ...) with b_slices
 * 1 (shared) or batch.  No counterpart in the reference's units: a cache of the operand split
 * that this build's GEMM performs. */
size_t cm_matmul_b_planes_bytes(uint32_t k, uint32_t m, uint32_t b_slices);
int cm_matmul_split_b(const int16_t* b, void* planes, uint32_t k, uint32_t m, uint32_t b_slices, int64_t b_bs,
                      uint32_t b_packed, uint32_t gemv_kw, void* stream);
int cm_matmul_planes(const int16_t* a, const void* b_planes, int16_t* c, uint32_t n, uint32_t k, uint32_t m,
                     uint32_t batch, int64_t a_bs, uint32_t b_slices, int64_t c_bs, uint32_t wrap32, void* stream);

/* cm_matmul_planes with A also split already, by the kernel that produced it
 * (cm_rowops_chain_planes, cm_vectorop_planes, cm_attention_planes): one slice, k a multiple
 * of 64, C = A . B as cm_matmul(a, b, c, n, k, m, 1, 0, 0, 0, ..., wrap32) computes it from the
 * int16 A those planes came from.  a_planes: cm_matmul_a_planes_bytes(n, k, nsum) bytes, 256-byte
 * aligned -- hi and lo byte planes [lines][k] (x - 128 = 256 hi + lo, lo with its top bit
 * flipped; lines = n rounded up to 256) and nsum partial row-sum arrays [nsum][lines] adding
 * up to each row's sum.  No counterpart in the reference: the operand split of this build's
 * matmul, done by the operand's producer. */
size_t cm_matmul_a_planes_bytes(uint32_t n, uint32_t k, uint32_t nsum);
int cm_matmul_aplanes(const void* a_planes, uint32_t nsum, const void* b_planes, int16_t* c, uint32_t n, uint32_t k,
                      uint32_t m, uint32_t wrap32, void* stream);

/* ---------------------------------------------------------------- Conv
 * Replaces ConvKernel (kernels/conv_rtl/model/include/ConvKernel.h:229-259) and the
 * simulator's Conv branches (_simulate.py:121-220, 643-660, 784-812): NCHW x, packed
 * weights (ConvKernel.h:136-159: [out_ch][ceil(in_ch/16)][kh][kw][16 or 8 lanes];
 * depthwise [out_ch][roundup(kh*kw, 8)]), bias [roundup(out_ch, 8)] when has_bias,
 *   y = sat16(floor((bias << 8 + sum x*w) / 2^8))  (wrap32: the sum wraps to int32 first),
 * implicit zero padding, and the y channel pattern: channel c's plane at
 * (c mod y_cn)*y_cs + (c div y_cn)*y_gs (y_cs = 0: out_h*out_w, y_cn = 0: one group;
 * batch must be 1 when either is set).  kh, kw <= 7 (the unit's bound). */
int cm_conv(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
            uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
            uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
            uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
            uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs,
            uint32_t y_cn, uint32_t y_gs, uint32_t wrap32, void* stream);

/* Constant weights of a standard (not depthwise) convolution split once: cm_conv_split_w
 * writes the byte planes and row sums of the packed weights w -- what every cm_conv call
 * otherwise derives from w on the fly -- into `planes` (cm_conv_w_planes_bytes(out_ch, in_ch,
 * kh, kw) bytes, 256-byte aligned); cm_conv_planes, with cm_conv's arguments otherwise
 * (is_depthwise 0), then computes exactly cm_conv.  No counterpart in the reference's units:
 * a cache of the operand split that this build's GEMM performs. */
size_t cm_conv_w_planes_bytes(uint32_t out_ch, uint32_t in_ch, uint32_t kh, uint32_t kw);
int cm_conv_split_w(const int16_t* w, void* planes, uint32_t out_ch, uint32_t in_ch, uint32_t kh, uint32_t kw,
                    void* stream);
int cm_conv_planes(const int16_t* x, const void* w_planes, const int16_t* bias, int16_t* y,
                   uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
                   uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
                   uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                   uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs,
                   uint32_t y_cn, uint32_t y_gs, uint32_t wrap32, void* stream);

/* cm_conv / cm_conv_planes with the VectorOP activation that follows the conv in the graph
 * applied to the result before it is stored: act 1 = RELU (VectorOP op 4), 2 = RELU6 (op 5,
 * clamp of the raw int16 to [0, 6 * 2^8]), 0 = none; CM_EINVAL for any other act.  No
 * counterpart in the reference's units (the reference runs the activation as its own VectorOP
 * call, nodes.py:395-441): a fusion of two unit calls into one, with the second call's exact
 * result. */
int cm_conv_act(const int16_t* x, const int16_t* w, const int16_t* bias, int16_t* y,
                uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
                uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
                uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs,
                uint32_t y_cn, uint32_t y_gs, uint32_t wrap32, uint32_t act, void* stream);
int cm_conv_planes_act(const int16_t* x, const void* w_planes, const int16_t* bias, int16_t* y,
                       uint32_t batch, uint32_t in_ch, uint32_t in_h, uint32_t in_w, uint32_t out_ch,
                       uint32_t out_h, uint32_t out_w, uint32_t kh, uint32_t kw, uint32_t stride_h,
                       uint32_t stride_w, uint32_t dilation_h, uint32_t dilation_w, uint32_t pad_top,
                       uint32_t pad_left, uint32_t has_bias, uint32_t is_depthwise, uint32_t y_cs,
                       uint32_t y_cn, uint32_t y_gs, uint32_t wrap32, uint32_t act, void* stream);

/* ---------------------------------------------------------------- Pooling
 * Replaces PoolingKernel (kernels/pool_rtl/model/include/PoolingKernel.h:120-140) and the
 * simulator's pool reference (_simulate.py:230-358, 701-719): pool_type 0 MAX, 1 AVG
 * (sum * round(2^23/d) >> 23), 2 LP (lp_order 1: sum |x|; 2: the polynomial square root);
 * NCHW in and out. */
int cm_pool(const int16_t* x, int16_t* y, uint32_t batch, uint32_t channels, uint32_t in_h,
            uint32_t in_w, uint32_t out_h, uint32_t out_w, uint32_t pool_h, uint32_t pool_w,
            uint32_t stride_h, uint32_t stride_w, uint32_t pad_top, uint32_t pad_left,
            uint32_t dil_h, uint32_t dil_w, uint32_t pool_type, uint32_t lp_order,
            uint32_t count_include_pad, void* stream);

/* ---------------------------------------------------------------- RowOps
 * Replaces one RowOpsKernel job: the register block of
 * doc/kernels/ROWOPS_RTL_KERNEL.md section 1.2 (driven by run_rowops,
 * inference-scheduler/src/rowops_nodes.py:143-151) with the integer specifications of
 * inference-scheduler/src/rowops_spec.py.  a, b, c, p are device byte addresses (the
 * registers 0x20 / 0x30 / 0x40 / 0x50), every stride in BYTES; op carries the code [3:0],
 * the kinds and the flags (B_EN, P_BCAST, P_KEEP, RELU, NORM_LN, SCALE).  Row outputs
 * are whole 16-byte words, the lanes past n written 0 (TRANSPOSE with scattered granules
 * writes exactly its granules).  The parameter RAM is emulated per device: a job that
 * loads parameters copies its block into it, a P_KEEP job reads what the last load left.
 * TLOAD (op 8) loads the table image from `a` (4096 int32 words in order).  Every other job
 * with work to do writes c: a null c is refused (CM_EINVAL). */
int cm_rowops(const void* a, const void* b, void* c, const void* p, uint32_t op, uint32_t n,
              uint32_t c1, uint32_t c2, uint32_t a_s1, uint32_t a_s2, uint32_t b_s1,
              uint32_t b_s2, uint32_t c_s1, uint32_t c_s2, int64_t eps, uint32_t aux,
              uint32_t bq_sh, uint32_t win_lo, uint32_t win_hi, void* stream);

/* One row-ops descriptor (ROWOPS_RTL_KERNEL.md section 1.6: the argument registers
 * 0x10 .. 0x6C in register order), pointers as device addresses. */
typedef struct cm_rowops_desc {
    uint32_t op, n, c1, c2;
    uint64_t a;
    uint32_t a_s1, a_s2;
    uint64_t b;
    uint32_t b_s1, b_s2;
    uint64_t c;
    uint32_t c_s1, c_s2;
    uint64_t p;
    int64_t eps;
    uint32_t aux, bq_sh, win_lo, win_hi;
} cm_rowops_desc;

/* A descriptor chain: the jobs of a HOST array in order on `stream`, each reading what
 * the previous ones wrote (ROWOPS_RTL_KERNEL.md section 1.6; no 16-job cap). */
int cm_rowops_chain(const cm_rowops_desc* jobs, uint32_t n_jobs, void* stream);

/* cm_rowops_chain that also writes the byte planes of the last job's output for a following
 * cm_matmul_aplanes (A = that output): the last job is a NORM of int16 rows of n elements, n a
 * multiple of 64, with its own parameter block; `planes` holds cm_matmul_a_planes_bytes(c1 c2,
 * n, ceil(n / 1024)) bytes, 256-byte aligned (row r of the job grid = i2 c1 + i1).  That
 * NORM's c may be 0 when only the matmul reads its rows (the planes alone are written); any
 * other null output is refused (CM_EINVAL).  In both
 * chain calls a COPY / ADDX job with an int32 output that the next job, a NORM over the same
 * rows, takes as its A runs with that NORM as one launch (each row read once; the parameter
 * RAM ends as the NORM leaves it).  No counterpart in the reference: the chain of
 * ROWOPS_RTL_KERNEL.md section 1.6, with the operand split of this build's matmul folded into
 * the NORM that produces the operand. */
int cm_rowops_chain_planes(const cm_rowops_desc* jobs, uint32_t n_jobs, void* planes, void* stream);

/* ---------------------------------------------------------------- Layout
 * The attention's operand moves between the projection MatMuls and the contractions (the
 * reference does them on the host / by DMA: VitAttnPrep and LlmAttnMerge, vit.py:19-32,
 * llm_nodes.py AttnPrep / Merge): a 4-D strided int16 gather,
 *   dst[i0][i1][i2][i3] (contiguous) = src[i0 * s0 + i1 * s1 + i2 * s2 + i3 * s3]
 * (strides in elements).  No unit of the reference's five; the exact copy of its moves. */
int cm_permute16(const int16_t* src, int16_t* dst, uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
                 uint64_t s0, uint64_t s1, uint64_t s2, uint64_t s3, void* stream);

/* dst[i0 t0 + i1 t1 + i2 t2 + i3 t3] = src[i0 s0 + i1 s1 + i2 s2 + i3 s3] for i_k < d_k (elements):
 * cm_permute16 into a strided destination, e.g. the step's K / V rows into the group-major
 * caches [KV][C][HD] at row pos (the cache writes of LlmAttnPrep / AttnPrepRoNode,
 * llm_nodes.py:1012-1030, rowops_nodes.py:1114).  src and dst must not overlap. */
int cm_copy16(const int16_t* src, int16_t* dst, uint32_t d0, uint32_t d1, uint32_t d2, uint32_t d3,
              uint64_t s0, uint64_t s1, uint64_t s2, uint64_t s3, uint64_t t0, uint64_t t1, uint64_t t2,
              uint64_t t3, void* stream);

/* The token-id embedding lookup of LlmEmbedNode (inference-scheduler/src/llm_nodes.py:466-570), a
 * gather: out[t][0 .. d) = table[clamp(ids[t], 0, rows - 1)][0 .. d) for t < n_ids, out of 32-bit
 * lanes.  `table` holds the output's own lanes for every row -- the int32 residual's raws
 * (table_i16 = 0, or table_i16 = 1 for int16 raws that the gather sign-extends, the reference's
 * int16 storage of a residual table whose raws fit) or float32 values (table_i16 = 0) -- so the
 * gather is exact.  d a multiple of 4, `out` 16-byte aligned, table rows 16-byte (int16: 8-byte)
 * aligned; ids int32 on the device. */
int cm_embed_rows(const void* table, uint32_t table_i16, const int32_t* ids, void* out, uint32_t n_ids,
                  uint32_t rows, uint32_t d, void* stream);

/* ---------------------------------------------------------------- Attention (composed)
 * The attention of an encoder layer in one call -- no counterpart among the reference's
 * units: the composition of VitAttnPrep (head split), the q.K^T contraction (the arithmetic
 * of LlmAttnConvNode, int32 wrap), VitAttnSoftmaxVopNode's keys-major softmax (VectorOP op 11,
 * every key valid), the P.V contraction and the head merge (vit.py:19-32,
 * llm_nodes.py:995-1001 and 1407-1425, smx_nodes.py:121-248), exactly as those calls in turn
 * compute it.  For sequence b of `batch` (seq tokens, rows of qkv ld elements apart from
 * qkv + b*seq*ld) and head h of `heads` (head_dim 64): Q, K, V at columns q_off, k_off, v_off
 * + 64 h; s[j][i] = sat16(wrap32(K[j].Q[i]) >> 8); P[i][.] = the softmax unit over the keys of
 * query i with smx_cm / smx_cfg; o[i][d] = sat16(wrap32(sum_j P[i][j] V[j][d]) >> 8), written to
 * o + (b*seq + i)*o_ld + 64 h + d.  seq in {64, 128, 256, 384}; 16-byte aligned rows and
 * column offsets. */
int cm_attention(const int16_t* qkv, int16_t* o, uint32_t batch, uint32_t seq, uint32_t heads, uint32_t head_dim,
                 uint64_t ld, uint32_t q_off, uint32_t k_off, uint32_t v_off, uint64_t o_ld, uint32_t smx_cm,
                 uint32_t smx_cfg, void* stream);

/* cm_attention with o's rows exactly heads x 64 wide (o_ld = heads * 64), also writing o's byte
 * planes for the output projection (cm_matmul_aplanes with A = o: n = batch * seq, k = heads *
 * 64, nsum = heads): `planes` holds cm_matmul_a_planes_bytes(batch * seq, heads * 64, heads)
 * bytes, 256-byte aligned; o may be NULL when only the projection reads it (the planes alone
 * are written).  No counterpart in the reference: the operand split of this build's matmul,
 * done by the attention that produces the operand. */
int cm_attention_planes(const int16_t* qkv, int16_t* o, uint32_t batch, uint32_t seq, uint32_t heads,
                        uint32_t head_dim, uint64_t ld, uint32_t q_off, uint32_t k_off, uint32_t v_off,
                        uint32_t smx_cm, uint32_t smx_cfg, void* planes, void* stream);

/* One decode step's attention, fused, for `groups` KV groups: group bg's g query rows q[bg g +
 * i][0..hd) against its cache rows kc / vc[bg c + j][0..hd) (head_dim hd 32 or 64, c a
 * multiple of 64 up to 8192, g <= 8),
 *   s[i][j] = sat16(wrap32(sum_d q[i][d] kc[j][d]) >> 8),
 *   P[i][.] = the softmax unit's row mode over s[i][.] (cm_vectorop op 10 with smx_cm / smx_cfg /
 *             smx_mask; the softmax row index of (bg, i) is bg g + i),
 *   o[bg g + i][d] = sat16(wrap32(sum_j P[i][j] vc[j][d]) >> 8).
 * The chain of two cm_matmul wrap contractions around a cm_vectorop softmax, as the reference
 * runs a decode step's q.K^T, softmax and P.V (llm_nodes.py:1183-1425, vectorop_smx.py:50-66);
 * no counterpart as one unit call.  16-byte aligned operands. */
int cm_decode_attention(const int16_t* q, const int16_t* kc, const int16_t* vc, int16_t* o, uint32_t groups,
                        uint32_t g, uint32_t c, uint32_t head_dim, uint32_t smx_cm, uint32_t smx_cfg,
                        uint32_t smx_mask, void* stream);

/* A decode step's attention prep in one launch (no counterpart as one unit call): the ROPE jobs
 * of q [batch][heads hd] and k [batch][kv_heads hd] at one position -- op words op_q / op_k
 * (int16 A and C, the int32 table as B), their 16-byte parameter blocks params_q / params_k,
 * rope_row the table row of the position (cos [hd] then sin [hd], int32) -- with q's result
 * into qr and k's straight into the K cache rows kc[b][g][pos][0..hd), and v's rows copied into
 * vc[b][g][pos] (caches [batch][kv_heads][cache_rows][hd]): the cm_rowops ROPE jobs and the two
 * KV row writes of the reference's attention prep (rowops_nodes.py:997-1047, llm_nodes.py:
 * 1012-1030) with the same element rule.  hd a multiple of 16 up to 128, 16-byte aligned rows
 * and rope_row.
 * The device's row-ops parameter RAM is left as it was. */
int cm_decode_prep(const int16_t* q, const int16_t* k, const int16_t* v, int16_t* qr, int16_t* kc, int16_t* vc,
                   uint32_t batch, uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t cache_rows,
                   uint32_t pos, const void* rope_row, const void* params_q, uint32_t op_q, const void* params_k,
                   uint32_t op_k, void* stream);

/* cm_decode_prep followed by cm_decode_attention over its outputs, in one launch: the prep of
 * each KV group done by that group's attention workgroup before its q.K^T (the group's query
 * heads into qr, its K / V cache rows at pos), then o as cm_decode_attention(qr, kc, vc, o,
 * batch kv_heads, heads / kv_heads, cache_rows, head_dim, smx_cm, smx_cfg, smx_mask) computes it.
 * No counterpart in the reference: its RoPE / KV-write nodes and the attention chain, one launch. */
int cm_decode_attention_prep(const int16_t* q, const int16_t* k, const int16_t* v, int16_t* qr, int16_t* kc,
                             int16_t* vc, int16_t* o, uint32_t batch, uint32_t heads, uint32_t kv_heads,
                             uint32_t head_dim, uint32_t cache_rows, uint32_t pos, const void* rope_row,
                             const void* params_q, uint32_t op_q, const void* params_k, uint32_t op_k,
                             uint32_t smx_cm, uint32_t smx_cfg, uint32_t smx_mask, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CORMORANT_HIP_H */
