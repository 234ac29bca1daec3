/*
 * qlinear.h -- C ABI of the MI355X (gfx950) quantized decode linear-layer library.
 *
 * Plain pointers and sizes only. Every pointer argument is device memory (HBM) unless
 * it says otherwise; `stream` is a hipStream_t (NULL = the default stream). No entry
 * point allocates, synchronises or reads device memory on the host, so every call is safe to
 * capture into a hipGraph. Each
 * returns QLX_OK (0) or a negative status; qlx_last_error() then holds a message
 * (thread-local).
 *
 * Number formats travel as raw bits: bf16 and fp16 as uint16, OCP e4m3fn as one byte.
 *
 * The reference binds its kernels through ctypes to the CUDA driver
 * (engine/kernels/cuda_jit.py:141-289, cuLaunchKernel with arrays of c_void_p/c_int);
 * each function below replaces one Python-level operator of engine/kernels, cited per
 * entry. The Python shims in dryft-flash-infer_amd/kernels keep the reference names.
 */
#ifndef QLINEAR_H
#define QLINEAR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QLX_ABI_VERSION 1

/* status codes */
#define QLX_OK 0
#define QLX_EINVAL (-1) /* contract violation, detected before any launch */
#define QLX_EHIP (-2)   /* HIP runtime error */

/* scale_kind */
#define QLX_SCALE_F16 0
#define QLX_SCALE_BF16 1

/* storage */
#define QLX_STORE_OFFSET 0 /* q + offset (128 or 8) as one uint8 per value */
#define QLX_STORE_SIGNED 1 /* q as int8 */
#define QLX_STORE_K32 2    /* int4 codes q + 8, eight per int32 along K: nibble i of word j is k = 8j+i */

/* linear modes */
#define QLX_MODE_BF16 0   /* y[m][n] bf16 */
#define QLX_MODE_PLANES 1 /* fp32 split-K planes [splits][m][n], not reduced */
#define QLX_MODE_SWIGLU 2 /* weight rows = [gate; up] (2I), y[m][i] = bf16(bf16(silu(g)) * u) */

/* Launch plan of a linear call. `splits` K-slices run as separate workgroups; with
 * splits > 1 and mode != PLANES the last workgroup of each row block sums the slices in
 * slice order (deterministic) from `workspace` ([splits][m][n] fp32) and finishes the
 * epilogue, using `tickets` (>= qlx_plan_tickets(plan) int32, zero before the first call;
 * every call leaves them zero again). Calls that share `tickets` must not overlap. */
typedef struct qlx_plan {
  int mode;         /* QLX_MODE_* */
  int splits;       /* K slices, >= 1 */
  int waves;        /* waves per workgroup: 4 or 8 */
  int kw;           /* waves per 16-row tile (1, 2, 4 or 8; divides waves) */
  int rw;           /* 16-row tiles per wave (1 or 2), reusing each activation fragment */
  float* workspace; /* fp32 [splits][m][n] (mode PLANES: the output planes) */
  int* tickets;     /* per-row-block counters */
} qlx_plan;

const char* qlx_last_error(void);
int qlx_abi_version(void);

/* ---- quantize / pack / relayout (load time) ------------------------------------- */

/* Symmetric absmax weight quantize of bf16 w[rows][k], one scale per `group` values.
 * Replaces cuda_fp8.quantize (engine/kernels/cuda_fp8.py:1127-1151): the defaults of that
 * function are scale_kind=F16, nudge=1, storage=OFFSET. The north-star formats are
 * W8A16 per-channel (group=k, BF16, SIGNED) and W4A16 (group=128, BF16, K32).
 * data: uint8/int8 [rows][k], or int32 [rows][k/8] for K32; scale: [rows][k/group]. */
int qlx_quantize_weight(const void* w, void* data, void* scale, int rows, int k, int group,
                        int bits, int scale_kind, int nudge, int storage, void* stream);

/* bf16((q - offset) * scale) -> out[rows][k]. Replaces cuda_fp8.dequantize
 * (engine/kernels/cuda_fp8.py:1154-1161). */
int qlx_dequantize(const void* data, const void* scale, void* out, int rows, int k, int groups,
                   int bits, int scale_kind, int storage, void* stream);

/* cuda_fp8.Prepared weight layout (engine/kernels/cuda_fp8.py:1164-1205): tiled 8-bit,
 * row-major fragment-permuted 8-bit (tiled=0), or tiled 4-bit nibbles. */
int qlx_prepare_ref(const void* data, void* out, int rows, int k, int bits, int tiled, void* stream);

/* Prepared.row_major for the tiled 8-bit layout (engine/kernels/cuda_fp8.py:1207-1214). */
int qlx_row_major_ref(const void* weight, void* out, int rows, int k, void* stream);

/* E4M3 weight quantize, bf16 scales per `group` (engine/kernels/fp8.py:20-28).
 * group = k is the per-output-channel FP8 W8A8 weight. */
int qlx_quantize_fp8_weight(const void* w, void* code, void* scale, int rows, int k, int group,
                            void* stream);

/* Dynamic per-token e4m3 activation quantize: scale[m] = max(amax/448, 1e-12) (fp32),
 * code = e4m3(clamp(x/scale, +-448)). The W8A8 path of cuda_int8.quantize_activation
 * (engine/kernels/cuda_int8.py:58-88) with the north star's FP8 per-token granularity. */
int qlx_quantize_fp8_act(const void* x, void* code, float* scale, int m, int k, void* stream);

/* Exhaustive check of the arithmetic every FP8 quantizer here shares (weights, activations,
 * in-kernel prologues): for each bf16 maximum (finite or +inf), its scale max(amax/448, 1e-12)
 * and every bf16 value of no larger magnitude (plus every NaN), the fast code path against
 * IEEE division + clamp + RNE cast. No counterpart in the reference; a diagnostic for tests.
 * counts: 66 zeroed uint64 in device memory; counts[0] = mismatches, counts[1] = recorded,
 * counts[2..65] = (amax bits << 48 | x bits << 32 | fast code << 8 | reference code). */
int qlx_fp8_selfcheck(unsigned long long* counts, void* stream);

/* cuda_int8.Prepared weight (engine/kernels/cuda_int8.py:100-108) from the fragment-permuted
 * row-major bytes. */
int qlx_int8_prepare(const void* row_major_ref, void* out, int rows, int k, void* stream);

/* cuda_int8.quantize_activation (engine/kernels/cuda_int8.py:58-88): q int8 [m][k] in
 * fragment order, scale fp32 [m][k/64]; with q2 != NULL also the residual component
 * (components=2). */
int qlx_quantize_act_int8(const void* x, void* q, float* scale, void* q2, float* scale2, int m, int k,
                          void* stream);

/* MI355X tile layout of a row-major [rows][row_bytes] weight (rows % 16 == 0, row_bytes %
 * 128 == 0): the 16-row x 128-byte block (tile t, step s) is stored contiguously at
 * (t * row_bytes/128 + s) * 2048, ordered [j 2][c 4][r 16][16 bytes] = row 16t + r, bytes
 * 128s + 64j + 16c -- the order a wave's loads consume it, so every load instruction reads
 * 1 KB of consecutive bytes. The load-time relayout counterpart of cuda_fp8.Prepared's tiles
 * (engine/kernels/cuda_fp8.py:1183-1205). */
int qlx_tile_rows(const void* src, void* dst, int rows, int row_bytes, void* stream);

/* ---- linear layers: y = x . W^T (x bf16 [m][k] unless stated) ------------------------ */
/* The north-star linears take `tiled` = 1 for a weight relaid by qlx_tile_rows, 0 for the
 * row-major packed weight. */

/* Default plan for a linear call (the selection the reference races in
 * engine/kernels/gemm.py:134-261 / cuda_fp8._plan:1255-1276). fmt is one of QLX_FMT_*. */
#define QLX_FMT_W8A16 0   /* int8 [n][k] signed, bf16 scale [n] */
#define QLX_FMT_W4A16 1   /* int32 [n][k/8] k32 codes, bf16 scale [n][k/128] */
#define QLX_FMT_FP8 2     /* e4m3 [n][k], bf16 scale [n], x quantized per token in-kernel */
#define QLX_FMT_REF8 3    /* cuda_fp8 8-bit: offset bytes, fp16 scale [n][k/64] */
#define QLX_FMT_REF4 4    /* cuda_fp8 4-bit tiled nibbles, fp16 scale [n][k/64] */
#define QLX_FMT_FP8WO 5   /* fp8.fp8_matmul: e4m3 [n][k], bf16 scale [n][k/group], x bf16 */
#define QLX_FMT_INT8 6    /* cuda_int8: int8 [n][k] fragment order, fp16 scale [n][k/64] */
int qlx_plan_linear(int fmt, int mode, int m, int n, int k, qlx_plan* plan);
int qlx_plan_tickets(const qlx_plan* plan, int fmt, int m, int n, int k);
/* Normalise plan->splits so every K slice is non-empty; with `grow`, first raise it until the
 * plan's LDS fits (the reference's _plan, engine/kernels/cuda_fp8.py:1255-1276). comp =
 * activation components (2 only for QLX_FMT_INT8 with a residual component). */
int qlx_plan_fit(qlx_plan* plan, int fmt, int m, int n, int k, int comp, int grow);

/* W8A16 per output channel. Replaces the W8A16 call of cuda_fp8.matmul
 * (engine/kernels/cuda_fp8.py:1316-1330) for the north-star per-channel format. */
int qlx_linear_w8a16(const void* w, const void* w_scale, const void* x, void* y, int m, int n,
                     int k, int tiled, const qlx_plan* plan, void* stream);

/* W4A16, group-128 bf16 scales, int32 k32 words. Replaces cuda_fp8.matmul / matmul_partials /
 * gate_up_swiglu at bits=4 (engine/kernels/cuda_fp8.py:1307-1330, 1381-1390). */
int qlx_linear_w4a16(const void* w, const void* w_scale, const void* x, void* y, int m, int n,
                     int k, int tiled, const qlx_plan* plan, void* stream);

/* Skinny GEMM for 16..64 tokens (speculative verification, small batches), W4A16 or W8A16
 * in the MI355X tile layout: the activation streams through LDS one K step at a time, shared
 * by a workgroup's waves; K slices (plan->splits > 1) write fp32 planes to plan->workspace
 * ([splits][m][n]) that are reduced in slice order: with plan->tickets (>= n/16 int32, zero
 * before the first call, left zero by every call; calls sharing them must not overlap) by the
 * last workgroup of each row group in the same launch, else by a second launch
 * (qlx_reduce_planes, or qlx_swiglu for mode SWIGLU) -- the same sums either way, bit-identical.
 * W4A16 batches of 33..64 tokens on 4-wave plans may run as two token blocks of at most 32
 * (one K slice over more than 256 row groups; or K slices without tickets whose two blocks fit
 * 512 workgroups): bit-identical output, chosen inside the call (skinny.hip).
 * Same arithmetic as qlx_linear_w4a16 / qlx_linear_w8a16.
 * Serves the batches the reference runs through cuda_fp8.matmul's 8-token tiles
 * (engine/kernels/cuda_fp8.py:1227-1234, 1316-1330). qlx_plan_skinny fills waves (4 or 8)
 * and splits for a shape. */
int qlx_plan_skinny(int fmt, int mode, int m, int n, int k, qlx_plan* plan);
int qlx_linear_skinny(int fmt, const void* w, const void* w_scale, const void* x, void* y, int m, int n, int k,
                      const qlx_plan* plan, void* stream);

/* The skinny GEMM for FP8 W8A8 at 9..64 tokens: the activation quantized per token beforehand
 * (qlx_quantize_fp8_act or qlx_add_norm_quant_fp8: e4m3 codes [m][k] and fp32 scales [m]), its
 * codes streamed through LDS per K step against e4m3 weights on the fp8 MFMA; each output is
 * the fp32 product times the channel's and the token's scale (qlx_plan_skinny with
 * QLX_FMT_FP8 plans it). The W8A8 batches the reference serves through cuda_int8.matmul at
 * b9-16 (engine/kernels/cuda_int8.py:251-281; engine/engine.py:623-625). */
int qlx_linear_skinny_fp8(const void* w, const void* w_scale, const void* x_code, const float* x_scale, void* y,
                          int m, int n, int k, const qlx_plan* plan, void* stream);

/* qlx_linear_skinny for callers that cannot allocate (code under graph capture, serving
 * loops, harnesses that forbid hipMalloc): no counterpart in the reference. It plans the call
 * itself (qlx_plan_skinny) and keeps the K-slice planes and ticket counters in the library's
 * own static device array (8 MiB of planes + 16384 counters per GPU, held until the process
 * ends) instead of caller memory; it calls no hipMalloc/hipFree. Rejects (QLX_EINVAL) shapes
 * whose planes (splits * m * n * 4 bytes) exceed 8 MiB or with n > 262144. Every call on one
 * GPU shares that array: calls that overlap on one GPU (other streams, other threads) race.
 * Same output as qlx_linear_skinny with the same plan, bit for bit. */
int qlx_linear_skinny_noalloc(int fmt, const void* w, const void* w_scale, const void* x, void* y, int m, int n,
                              int k, int mode, void* stream);

/* FP8 e4m3 W8A8: per-channel bf16 weight scales, activation quantized per token inside the
 * kernel (same arithmetic as qlx_quantize_fp8_act). Replaces cuda_int8.matmul's role
 * (engine/kernels/cuda_int8.py:251-281) for the north-star FP8 format. */
int qlx_linear_fp8_w8a8(const void* w, const void* w_scale, const void* x, void* y, int m, int n,
                        int k, int tiled, const qlx_plan* plan, void* stream);

/* qlx_linear_fp8_w8a8 on an activation qlx_quantize_fp8_act quantized beforehand (e4m3 codes
 * [m][k], fp32 token scales [m]; K a multiple of 128): bit-identical results, one quantization
 * per projection instead of one per workgroup. */
int qlx_linear_fp8_w8a8_q(const void* w, const void* w_scale, const void* x_code, const float* x_scale, void* y,
                          int m, int n, int k, int tiled, const qlx_plan* plan, void* stream);

/* cuda_fp8.matmul / matmul_partials / gate_up_swiglu on the reference's own Prepared weights
 * (engine/kernels/cuda_fp8.py:1279-1330, 1381-1390): bits 8 (tiled or row-major) or 4. */
int qlx_linear_ref(const void* w, const void* w_scale, const void* x, void* y, int m, int n,
                   int k, int bits, int tiled, const qlx_plan* plan, void* stream);

/* fp8.fp8_matmul: E4M3 weights with bf16 scales per `group` along K, bf16 activations
 * (engine/kernels/fp8.py:121-150). */
int qlx_linear_fp8wo(const void* w, const void* w_scale, const void* x, void* y, int m, int n,
                     int k, int group, const qlx_plan* plan, void* stream);

/* cuda_int8.matmul_quantized (engine/kernels/cuda_int8.py:251-276): int8 weights and
 * activations in fragment order, fp16 weight scales [n][k/64], fp32 activation scales
 * [m][k/64]; xq2/x_scale2 (or NULL) the optional residual component. */
int qlx_linear_int8(const void* w, const void* w_scale, const void* xq, const float* x_scale,
                    const void* xq2, const float* x_scale2, void* y, int m, int n, int k,
                    const qlx_plan* plan, void* stream);

/* y = x . W^T into `delta` (bf16 [m][n]), then in the same launch res_out = bf16(residual +
 * delta) and normed = bf16(bf16(res_out * rsqrt(mean res_out^2 + eps)) * norm_w) over rows of
 * n: the workgroup that completes the last row block finishes every row. fmt is
 * QLX_FMT_W8A16, QLX_FMT_W4A16 or QLX_FMT_FP8 (weights as their linears take them, `tiled`
 * as there) or QLX_FMT_REF8 / QLX_FMT_REF4 (the cuda_fp8 layouts; `tiled` as in
 * qlx_linear_ref). plan->mode must be QLX_MODE_BF16; splits > 1 use plan->workspace and
 * plan->tickets as the linears do. `counter` is one int32, zero before the first call and
 * left zero by every call: calls sharing it must not overlap. n % 8 == 0.
 * Replaces cuda_fp8.matmul_add_norm (engine/kernels/cuda_fp8.py:1333-1374, kernel 695-963). */
int qlx_linear_add_norm(int fmt, const void* w, const void* w_scale, const void* x, int m, int n, int k,
                        int tiled, const void* residual, const void* norm_w, float eps, void* delta,
                        int* counter, void* res_out, void* normed, const qlx_plan* plan, void* stream);

/* ---- split-K plane consumers and epilogues ----------------------------------------- */

/* out[i] = bf16(sum_s planes[s][i]), s in order. Replaces the reduce_partials kernel of
 * cuda_fp8.matmul (engine/kernels/cuda_fp8.py:965-981, 1324-1330). */
int qlx_reduce_planes(const float* planes, void* out, long long width, int splits, void* stream);

/* out[i] = bf16(x[i] + bf16(sum_s planes[s][i])). Replaces cuda_small.residual_partials
 * (engine/kernels/cuda_small.py:43-55, 154-160). */
int qlx_residual_planes(const void* x, const float* planes, void* out, long long width, int splits,
                        void* stream);

/* Residual add then RMSNorm over rows of n: res = bf16(x + delta) with delta bf16 [rows][n]
 * or bf16(sum of fp32 planes [splits][rows][n]); y = bf16(bf16(res * rsqrt(mean res^2 + eps)) * w).
 * delta = planes = NULL gives plain RMSNorm of x (res untouched). Replaces norm.add_rms_norm,
 * add_rms_norm_partials, rms_norm (engine/kernels/reference.py:13-28, norm.py:125-154,
 * cuda_small.py:57-87, 145-165). */
int qlx_add_rms_norm(const void* x, const void* delta, const float* planes, int splits, const void* w,
                     void* res, void* y, int rows, int n, float eps, void* stream);

/* Residual + RMSNorm + INT8 activation quantize (per 64-group, fragment order).
 * Replaces cuda_int8.add_norm_quant (engine/kernels/cuda_int8.py:17-55). */
int qlx_add_norm_quant_int8(const void* x, const void* delta, const float* planes, int splits,
                            const void* w, void* res, void* q, float* q_scale, int rows, int n, float eps,
                            void* stream);

/* Residual + RMSNorm + FP8 per-token activation quantize in one launch: r = bf16(x + delta)
 * (delta bf16 [rows][n], or fp32 planes [splits][rows][n] reduced in plane order; both NULL: r = x,
 * res not written), y = bf16(bf16(r * rsqrt(mean(r^2) + eps)) * w) (written if y != NULL), then
 * scale[row] = max(amax(y)/448, 1e-12) and code = e4m3(y / scale) as qlx_quantize_fp8_act gives
 * for y. The FP8 W8A8 counterpart of cuda_int8.add_norm_quant (engine/kernels/cuda_int8.py:17-55):
 * the next projection's activation arrives quantized (qlx_linear_fp8_w8a8_q). */
int qlx_add_norm_quant_fp8(const void* x, const void* delta, const float* planes, int splits, const void* w,
                           void* res, void* y, void* code, float* scale, int rows, int n, float eps, void* stream);

/* out[r][i] = bf16(bf16(silu(g)) * u) from bf16 gate_up [rows][2I] or fp32 planes
 * [splits][rows][2I] (g and u rounded to bf16 after the plane sum). Replaces swiglu.swiglu,
 * swiglu.swiglu_partials, cuda_small.swiglu_partials (engine/kernels/swiglu.py:12-64,
 * cuda_small.py:89-110). */
int qlx_swiglu(const void* gate_up, const float* planes, int splits, void* out, int rows, int inter,
               void* stream);

/* ---- decode-step executor ----------------------------------------------------------- */

/* One projection of a decode step: y = x @ deq(w)^T on tiled weights (qlx_tile_rows layout),
 * mode QLX_MODE_BF16 or QLX_MODE_SWIGLU. x is either memory that no projection of the chain
 * writes ([m][k], dense), or the y of an earlier projection -- all of it, or its first k
 * columns (x == that y, rows n_out apart) -- and is then read as that projection produces it.
 * kw: waves sharing one 16-row tile (1, 2, 4 or 8), or 0 for the planner. */
typedef struct qlx_stack_call {
  const void* w;
  const void* w_scale;
  const void* x;
  void* y;
  int n, k, mode, kw;
} qlx_stack_call;

/* Bytes of one device descriptor written by qlx_stack_build. */
int qlx_stack_desc_size(void);

/* Launch configuration of a chain, filled by qlx_stack_build, passed to qlx_stack_run. */
typedef struct qlx_stack_launch {
  int grid;        /* workgroups (one per CU per lane; the planner checks they fit at once) */
  int lds_bytes;   /* dynamic LDS per workgroup */
  int waves;       /* waves per workgroup */
  int desc_lds;    /* byte offset of the descriptors' LDS copy, or -1 (read from memory) */
  int lanes;       /* workgroup sets: lane l runs projections l, l + lanes, ... */
  int amax_off;    /* LDS byte offset of the per-token FP8 maxima (64 bytes) */
  int pieces;      /* 1 when a row block of the chain is cut into K pieces (the kernel with their
                      reduction, whose registers otherwise go to deeper weight prefetch), else 0 */
  int attention;   /* 1 when the chain has attention stages (qlx_stack_build_step), else 0 */
} qlx_stack_launch;

/* Plan a chain of `ncalls` projections of one format (W8A16, W4A16 or FP8 W8A8; m = 1..16)
 * for the executor: workgroups of `waves` (4 or 8) waves, `groups_per_cu` lanes of one
 * workgroup per CU (1..4; fewer if registers or LDS do not allow), lane l running projections
 * l, l + lanes, ... concurrently with the other lanes. Writes the descriptors to host memory `desc`
 * (ncalls * qlx_stack_desc_size() bytes; NULL to only size) and, if `plans` is not NULL, each
 * projection's plan (waves, kw; splits = the most K pieces of one row block). The chain keeps
 * published outputs and partial sums in `arena` (*arena_bytes of device memory, zeroed once
 * before the first run): call once with desc and arena NULL to size it, then again with both.
 * Outputs must not overlap each other or an input read from memory (EINVAL otherwise).
 * Replaces the reference's per-projection launches chained by programmatic dependent launch
 * inside a captured graph (engine/kernels/cuda_fp8.py:47-50, 150-169;
 * engine/kernels/cuda_jit.py:218-262): here the whole chain is one launch (at most 1024
 * workgroups). The arena's first 4096 bytes hold each workgroup's last run epoch (zero in a fresh
 * arena). */
int qlx_stack_build(int fmt, int m, const qlx_stack_call* calls, int ncalls, int waves, int groups_per_cu,
                    void* desc, qlx_plan* plans, void* arena, long long* arena_bytes, qlx_stack_launch* launch);

/* Run the chain: `desc` is the device copy of qlx_stack_build's descriptors, `launch` its
 * launch configuration and `arena` the arena they were built for (256-byte aligned). Each run
 * tags what it publishes with the next epoch after the one the arena holds (every workgroup
 * reads and stores its own copy), so the call has no per-run argument and captures into a
 * hipGraph (every replay is a new run). `error` is one int32 in device memory, zero before the
 * run: once a wait passes `budget_us` microseconds from the run's start, every wait gives up,
 * the first one writing (1 << kind) to it (0: an input from an earlier projection, 1: a
 * piece's partial sums), and that run's outputs are undefined. Runs sharing an arena must not
 * overlap (same stream, or ordered). */
int qlx_stack_run(int fmt, const void* desc, int ncalls, const qlx_stack_launch* launch, void* arena, int* error,
                  long long budget_us, void* stream);

/* ---- residual add + RMSNorm input stages of the decode-step executor ----------------- */

/* Residual add + RMSNorm input stage of an executor projection (the decode step's fused
 * residual consumer, engine/kernels/norm.py:125-139 with reference.py:13-28's casts). With norm_w
 * set, projection c's input is y = bf16(bf16(r * rsqrt(mean(r^2) + eps)) * norm_w) with
 * r = bf16(resid + delta) (r = resid when delta is NULL), and calls[c].x must be NULL. resid is
 * bf16 [m][k] in memory the chain does not write, or the resid_out of an earlier stage; delta is
 * NULL or the whole output y of an earlier projection. resid_out (optional) receives r and
 * normed_out (optional) y. For FP8 W8A8 the staged y is quantized per token like any input: the
 * norm -> FP8 activation quantize is fused. */
typedef struct qlx_norm_input {
  const void* resid;
  const void* delta;
  const void* norm_w;
  void* resid_out;
  void* normed_out;
  float eps;
  int pad;
} qlx_norm_input;

/* qlx_stack_build with residual add + RMSNorm input stages: where norms[c].norm_w is not
 * NULL, projection c's input is bf16(bf16(r * rsqrt(mean(r^2) + eps)) * norm_w) with
 * r = bf16(resid + delta) (r = resid without delta), computed inside the launch by every
 * workgroup with work in the projection; calls[c].x is NULL exactly then. `resid` is memory the
 * chain does not write or an earlier stage's resid_out; `delta` is the whole output of an
 * earlier projection; resid_out / normed_out (optional) receive r and the input (FP8 W8A8:
 * quantized per token over the normed row). A norm stage makes one pass over its rows: m * k <= 3 * 64 * waves * 8. norms may be NULL (= qlx_stack_build). Replaces
 * the reference's plane consumers and residual + RMSNorm kernels between projections
 * (engine/kernels/norm.py:53-80, 125-154; engine/kernels/cuda_small.py:43-87). */
int qlx_stack_build_normed(int fmt, int m, const qlx_stack_call* calls, int ncalls, const qlx_norm_input* norms,
                           int waves, int groups_per_cu, void* desc, qlx_plan* plans, void* arena,
                           long long* arena_bytes, qlx_stack_launch* launch);

/* An attention stage inside the executor's chain (one token: m = 1, batch 1; head_dim 128;
 * bf16 caches [1][n_kv][capacity][128]): per KV head, the per-head RMSNorm + RoPE of its query
 * heads and of the key, with the arithmetic of qlx_qkv_norm_rope (engine/kernels/rope.py:125-166),
 * the key and value written into the caches at the token's position p = positions[0], and
 * grouped-query attention over keys 0 .. p with the arithmetic of qlx_decode_attention
 * (engine/kernels/attention.py:37-178). It takes two consecutive chain entries:
 *   kind 1 (splits): calls[c].x = the whole output of an earlier projection (the fused qkv
 *     row: n_q query heads, then n_kv key heads, then n_kv value heads), calls[c].y = NULL,
 *     n = n_q * 128, k = (n_q + 2 * n_kv) * 128, w and w_scale NULL. `splits` work items per KV
 *     head, item s taking the 32-key blocks s, s + splits, ...; each publishes fp32 partials
 *     (maximum, total and accumulator per query row) inside the launch;
 *   kind 2 (merge): the entry right after, with the same attention fields; calls[c].x = NULL,
 *     calls[c].y = the attention output, bf16 [1][n_q * 128] (later projections may read it),
 *     n = n_q * 128, k = 0. One work item per query row combines the splits in order.
 * kind 0: calls[c] is a projection (as in qlx_stack_build_normed). The token is in the cos/sin
 * table when p < table_rows (else its query reads as NaN and nothing is written), and its key
 * and value are written when also p < capacity. Replaces the reference's head norm + RoPE
 * kernel and its split and merge attention kernels between the qkv and o projections of a
 * decode step (engine/engine.py:926-949). */
typedef struct qlx_stack_attention {
  int kind, n_q, n_kv, splits;
  int capacity, table_rows;
  const void* q_norm_w;  /* bf16 [128] */
  const void* k_norm_w;  /* bf16 [128] */
  const void* cos;       /* bf16 [table_rows][128] */
  const void* sin;
  const int* positions;  /* int32 device value: the token's position */
  void* k_cache;
  void* v_cache;
  float eps, scale;      /* RMSNorm epsilon; attention scale (head_dim^-0.5) */
} qlx_stack_attention;

/* qlx_stack_build_normed with attention stages: attns[c].kind selects what entry c is (attns
 * may be NULL: every entry a projection). */
int qlx_stack_build_step(int fmt, int m, const qlx_stack_call* calls, int ncalls, const qlx_norm_input* norms,
                         const qlx_stack_attention* attns, int waves, int groups_per_cu, void* desc,
                         qlx_plan* plans, void* arena, long long* arena_bytes, qlx_stack_launch* launch);

/* ---- QKV consumer and decode attention ----------------------------------------------- */

/* Arguments of qlx_qkv_norm_rope. Head dim is 128. Row r of the projection is token
 * r % seq_len of sequence r / seq_len; that token's position is positions[r % seq_len]. */
typedef struct qlx_rope_args {
  const void* qkv;        /* bf16 [rows][stride], or NULL when planes are given */
  const float* planes;    /* fp32 split-K planes [splits][rows][stride], or NULL */
  long long stride;       /* row width of qkv / planes, elements (multiple of 8) */
  int splits;
  int rows;
  int n_q;                /* Q heads normed and rotated into q_out (0: none) */
  int n_kv;               /* K heads normed, rotated and cached, V heads cached (0: none) */
  int q_col, k_col, v_col;/* column of head 0 of Q, K and V (multiples of 8) */
  int seq_len;
  int capacity;           /* cache slots per (sequence, KV head) */
  int table_rows;         /* rows of cos / sin */
  int pos_int64;          /* positions are int64 (else int32) */
  float eps;
  const void* q_norm_w;   /* bf16 [128] */
  const void* k_norm_w;   /* bf16 [128] */
  const void* cos;        /* bf16 [table_rows][128] */
  const void* sin;
  const void* positions;  /* [seq_len] */
  void* q_out;            /* bf16 [rows][n_q * 128] */
  void* k_cache;          /* bf16, or int8 with scales, [batch][n_kv][capacity][128] */
  void* v_cache;
  float* k_scale;         /* fp32 [batch][n_kv][capacity]: INT8 cache when non-NULL */
  float* v_scale;
  void* k_copy;           /* bf16 [batch][n_kv][seq_len][128] or NULL (prefill's SDPA input) */
  void* v_copy;
} qlx_rope_args;

/* Per-head RMSNorm + RoPE of Q and K, V copied, K/V written to cache slot positions[t]:
 * engine/kernels/rope.py:221-240 (qkv_norm_rope_to_cache), :200-218 (the split-K planes form),
 * :243-263 (q_norm_rope: n_kv = 0) and :266-297 (kv_norm_rope_to_cache: n_q = 0). One launch.
 * A position outside [0, table_rows) writes NaN to that row's Q heads and nothing to the
 * cache, as does one outside [0, capacity) for the cache. */
int qlx_qkv_norm_rope(const qlx_rope_args* args, void* stream);

/* Workspace bytes qlx_decode_attention needs for `splits` > 1 (0 for one split): the per-split
 * partials (no initial contents needed). */
int qlx_attention_workspace(int batch, int n_kv, int group, int tokens, int splits, size_t* bytes);

/* Grouped-query decode attention: engine/kernels/attention.py:282-315 (DecodeAttention.__call__,
 * the split and merge kernels :37-178). q bf16 [batch * tokens][n_kv * group *
 * 128]; caches [batch][n_kv][capacity][128] bf16, or int8 with fp32 scales [batch][n_kv]
 * [capacity]; pos (int32, device) is token 0's position: token t attends to keys 0 .. pos + t.
 * out bf16 like q. The live length is divided among `splits` workgroups per KV head on the
 * device, so the grid is fixed (capturable); with splits > 1 a second small kernel merges the
 * partials. Calls sharing a workspace must not overlap. tokens * group <= 64, head_dim 128. */
int qlx_decode_attention(const void* q, const void* k_cache, const void* v_cache, const float* k_scale,
                         const float* v_scale, const int* pos, void* out, void* workspace, size_t workspace_bytes,
                         int batch, int n_kv, int group, int head_dim, int tokens, int capacity, int splits,
                         float scale, void* stream);

/* ---- measurement ------------------------------------------------------------------- */

/* Read `bytes` (multiple of 16) from p with 16-byte loads over `blocks` workgroups of 256
 * threads, writing one word per workgroup to sink[blocks]: the HBM read floor the linears
 * are compared with (the reference's stream probe, bench/tiled_probe.py:20-31). */
int qlx_stream_read(const void* p, long long bytes, void* sink, int blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QLINEAR_H */
