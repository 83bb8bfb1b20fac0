/*
 * cannbench_amd.h - C ABI of the MI355X (gfx950) W8A8 MoE-FFN operator library.
 *
 * One C entry point per operator of the chain
 *
 *     AddRmsNormDynamicQuant -> GroupedMatmulSwigluQuant -> QuantMatmul / int8 GroupedMatmul
 *     (+ DynamicQuant)
 *
 * Conventions shared by every entry point:
 *   - Every tensor argument is a plain device pointer to a contiguous row-major buffer that the
 *     caller owns.  The library never allocates device memory; operators that need scratch memory
 *     take a `workspace` pointer sized by the matching *_workspace_size() query.
 *   - `group_list` is a HOST array of int64 cumulative row counts (the reference passes it as an
 *     `int[]` operator attribute): group g owns rows [group_list[g-1], group_list[g]), with
 *     group_list[-1] taken as 0.  Empty groups are allowed; group_list[E-1] must equal M.
 *   - Work is enqueued asynchronously on `stream` (a hipStream_t; NULL is the default stream).
 *     Nothing synchronises and nothing is read back to the host.
 *   - Every entry point validates its arguments first and returns a cb_status; on any error
 *     nothing is launched.  cb_status_string() gives the message, worded like the reference's
 *     TORCH_CHECK messages.
 *   - Entry points are reentrant: the only global state is a per-device property cache.
 */
#ifndef CANNBENCH_AMD_H
#define CANNBENCH_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  One per validation the reference performs with TORCH_CHECK. */
typedef enum cb_status {
    CB_OK = 0,
    CB_ERR_NULL_POINTER = 1,       /* a required pointer is NULL                               */
    CB_ERR_DTYPE = 2,              /* unsupported dtype code for this argument                 */
    CB_ERR_SHAPE = 3,              /* a dimension is negative or shapes disagree              */
    CB_ERR_K_MISMATCH = 4,         /* x.size(-1) != weight K                                  */
    CB_ERR_N_ODD = 5,              /* GroupedMatmulSwigluQuant needs an even N                */
    CB_ERR_GROUP_LEN = 6,          /* group_list length != expert count                       */
    CB_ERR_GROUP_COUNT = 7,        /* expert count outside [1, CB_MAX_EXPERTS]                */
    CB_ERR_GROUP_ORDER = 8,        /* group_list not a non-decreasing cumsum <= M             */
    CB_ERR_GROUP_TOTAL = 9,        /* group_list[-1] != M                                     */
    CB_ERR_SCALE_LEN = 10,         /* a scale / offset / bias has the wrong element count    */
    CB_ERR_ROW_TOO_LONG = 11,      /* AddRmsNormDynamicQuant row length > 16384               */
    CB_ERR_WORKSPACE = 12,         /* workspace missing or smaller than *_workspace_size()    */
    CB_ERR_EMPTY = 13,             /* QuantMatmul requires non-empty M, K, N                 */
    CB_ERR_LAUNCH = 14,            /* the HIP runtime refused a launch                       */
    CB_ERR_NO_DEVICE = 15,         /* no usable gfx950 device                                */
    CB_ERR_SCRATCH_LIMIT = 16      /* beyond the fixed scratch of a no-allocation entry point */
} cb_status;

/* dtype codes for the typed arguments. */
typedef enum cb_dtype {
    CB_DT_FLOAT16 = 1,
    CB_DT_BFLOAT16 = 2,
    CB_DT_FLOAT32 = 3,
    CB_DT_INT8 = 4,
    CB_DT_INT32 = 5,
    CB_DT_INT64 = 6
} cb_dtype;

/* Largest expert count accepted by the grouped operators (the reference accepts 64:
 * operators/groupedmatmulswigluquant/csrc/ops/grouped_matmul_swiglu_quant/op_kernel/gmsq_launch.h:35). */
#define CB_MAX_EXPERTS 256

/* Largest AddRmsNormDynamicQuant row length (the reference's limit,
 * operators/addrmsnormdynamicquant/csrc/ops/add_rms_norm_dynamic_quant/op_plugin/add_rms_norm_dynamic_quant_plugin.cpp:82-83). */
#define CB_ARDQ_MAX_ROW 16384

const char* cb_status_string(int status);

/* Library version string, e.g. "cannbench_amd 0.1 gfx950". */
const char* cb_version(void);

/*
 * Instrumentation (no reference counterpart): the next operator call made by this thread records
 * hipEvent_t `start_event` before and `stop_event` after its main kernel on the call's stream (the
 * GEMM kernel of the grouped / dense operators; all kernels of the row and routing operators), so a
 * caller can time the device work alone.  The setting is consumed by that call.  Either event may
 * be NULL.
 */
void cb_set_kernel_timing(void* start_event, void* stop_event);

/*
 * Measurement (no reference counterpart): the int8 matrix-core rate the device sustains.  Launches
 * 2 workgroups of 4 waves per CU, each wave issuing `iters` rounds of 8 independent
 * v_mfma_i32_32x32x32_i8 on register operands (no memory traffic), and stores the total operation
 * count (2 * 32 * 32 * 32 per MFMA) in *ops.  `sink` (at least 8 int32 per CU, device memory)
 * receives checksums that keep the work live.  Time it with cb_set_kernel_timing.
 * Returns CB_ERR_SHAPE for iters <= 0 or a short sink.
 */
int cb_probe_mfma_i8(int64_t iters, int32_t* sink, int64_t sink_len, int64_t* ops, void* stream);

/*
 * AddRmsNormDynamicQuant.
 * Replaces add_rms_norm_dynamic_quant(Tensor x1, Tensor x2, Tensor gamma, float epsilon)
 *   -> (Tensor y, Tensor xOut, Tensor scaleOut)
 * (operators/addrmsnormdynamicquant/csrc/ops/add_rms_norm_dynamic_quant/op_plugin/add_rms_norm_dynamic_quant_plugin.cpp:32,58-115)
 * and its launchers launch_ardq_half / launch_ardq_bf16 (add_rms_norm_dynamic_quant_launch.h:33-40).
 *
 *   x1, x2   : dtype [rows, row_len]        (dtype = CB_DT_FLOAT16 or CB_DT_BFLOAT16)
 *   gamma    : dtype [row_len]
 *   y        : int8  [rows, row_len]
 *   x_out    : dtype [rows, row_len]        x1 + x2 rounded to dtype
 *   scale_out: fp32  [rows]
 * rows == 0 or row_len == 0 returns CB_OK without a launch (the reference returns early).
 */
int cb_add_rms_norm_dynamic_quant(const void* x1, const void* x2, const void* gamma, int dtype,
                                  int64_t rows, int64_t row_len, float epsilon, int8_t* y,
                                  void* x_out, float* scale_out, void* stream);

/*
 * DynamicQuant (per-token symmetric int8).
 * Replaces dynamic_quant(Tensor x) -> (Tensor y, Tensor scale)
 * (operators/dynamicquant/csrc/ops/dynamic_quant/op_plugin/dynamic_quant_plugin.cpp:30,49-87).
 *   x: dtype [rows, row_len] (fp16 / bf16), y: int8 [rows, row_len], scale: fp32 [rows].
 */
int cb_dynamic_quant(const void* x, int dtype, int64_t rows, int64_t row_len, int8_t* y,
                     float* scale, void* stream);

/*
 * GroupedMatmulSwigluQuant.
 * Replaces grouped_matmul_swiglu_quant(Tensor x, Tensor weight, Tensor weight_scale,
 *   Tensor x_scale, int[] group_list) -> (Tensor y, Tensor y_scale)
 * (operators/groupedmatmulswigluquant/csrc/ops/grouped_matmul_swiglu_quant/op_plugin/gmsq_plugin.cpp:40-41,67-145)
 * and the launcher pair launch_gmsq_cube + launch_gmsq_vec (op_kernel/gmsq_launch.h:67-80).
 *
 *   x            int8 [M, K]        weight       int8 [E, K, N]  (N contiguous)
 *   weight_scale fp32 [E, N]        x_scale      fp32 [M]
 *   group_list   host int64 [group_len] cumulative counts
 *   y            int8 [M, N/2]      y_scale      fp32 [M]
 *   workspace    device bytes >= cb_grouped_matmul_swiglu_quant_workspace_size(M, K, N, E)
 * M == 0, N == 0 or E == 0 returns CB_OK without a launch (gmsq_plugin.cpp:93-95).
 */
int64_t cb_grouped_matmul_swiglu_quant_workspace_size(int64_t M, int64_t K, int64_t N, int64_t E);
int cb_grouped_matmul_swiglu_quant(const int8_t* x, const int8_t* weight, const float* weight_scale,
                                   const float* x_scale, const int64_t* group_list,
                                   int64_t group_len, int64_t M, int64_t K, int64_t N, int64_t E,
                                   int8_t* y, float* y_scale, void* workspace,
                                   int64_t workspace_bytes, void* stream);

/*
 * GroupedMatmulSwigluQuant with the activation rows gathered (no single reference counterpart: it
 * is the re-routing permutation of moe_re_routing, operators/moererouting/csrc/ops/moe_re_routing/
 * op_plugin/moe_re_routing_plugin.cpp:35-38, folded into the GEMM's activation loads, so the
 * permuted copy of the tokens is never written).  Routed row r (of M) computes with x row
 * row_index[r] and x_scale[row_index[r]]; x holds x_rows rows [x_rows, K] and x_scale x_rows
 * scales.  Output, group_list and workspace are those of cb_grouped_matmul_swiglu_quant for M rows,
 * and the results equal that operator on the gathered rows.  An index outside [0, x_rows) reads a
 * zero row with scale 0.  Requires x_rows * K < 2^31.
 */
int cb_grouped_matmul_swiglu_quant_gather(const int8_t* x, int64_t x_rows, const int32_t* row_index,
                                          const int8_t* weight, const float* weight_scale,
                                          const float* x_scale, const int64_t* group_list,
                                          int64_t group_len, int64_t M, int64_t K, int64_t N, int64_t E,
                                          int8_t* y, float* y_scale, void* workspace,
                                          int64_t workspace_bytes, void* stream);

/*
 * Diagnostics (no reference counterpart): the status word a GroupedMatmulSwigluQuant call left in
 * `workspace` (the same M, N, E).  0: every row-maximum exchange completed in time.  Bit 0: some
 * exchange wait gave up (its workgroups were not all resident together within the poll limit).
 * Bit 1: a decode-shaped tile was left to the fix-up launch without waiting, because waiting could
 * have depended on the waiting workgroup itself (only with few workgroups, e.g. a forced small
 * grid).  Either way the tiles concerned were recomputed by the fix-up launch with the final row
 * maxima, so the outputs are right and only time was lost.  Synchronises `stream`, so it is meant
 * for tests and debug runs, not the hot loop.  The status of cb_grouped_matmul_swiglu_quant_noalloc
 * calls is not readable: it lives in the library's hidden scratch array.
 */
int cb_grouped_matmul_swiglu_quant_status(const void* workspace, int64_t M, int64_t N, int64_t E,
                                          uint32_t* status, void* stream);

/*
 * GroupedMatmulSwigluQuant without a workspace argument and without any allocation.
 * No reference counterpart: for callers that cannot allocate device memory or pass a workspace
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, validation, results and stream behaviour as cb_grouped_matmul_swiglu_quant, with the
 * workspace taken from a fixed 4 MiB device array of the library (one per GPU, held until the
 * process ends; its address is looked up once per device on the first call there).  Problems whose
 * workspace would exceed 4 MiB return CB_ERR_SCRATCH_LIMIT (M = 131072 rows with N = 4096 and
 * E = 256 need about 0.7 MiB; the limit is reached near M = 979000).  Every call on one GPU shares
 * that GPU's array: calls that may overlap on one device (different streams, threads or
 * processes) race and must be ordered by the caller.  The exchange status word (see
 * cb_grouped_matmul_swiglu_quant_status) is kept in that array and cannot be queried.
 */
int cb_grouped_matmul_swiglu_quant_noalloc(const int8_t* x, const int8_t* weight, const float* weight_scale,
                                           const float* x_scale, const int64_t* group_list, int64_t group_len,
                                           int64_t M, int64_t K, int64_t N, int64_t E, int8_t* y,
                                           float* y_scale, void* stream);

/*
 * Test hook (no reference counterpart; for this library's tests only).  Overrides for the calling
 * thread's later launches, kept until changed; 0 restores each default:
 *   persistent_grid      workgroups of the persistent dequant / int32 GEMM and of the decode-shaped
 *                        GroupedMatmulSwigluQuant kernel (default: the CU count; a small grid makes
 *                        every workgroup walk many tiles); < 0 turns that
 *                        persistent launch off, and GroupedMatmulSwigluQuant then takes its
 *                        two-pass path (the one it takes when its fused grid cannot be resident).
 *   exchange_spin_limit  polls of the GroupedMatmulSwigluQuant row-maximum exchange before a tile
 *                        gives up and leaves its output to the fix-up launch (default 2^20, about
 *                        2 s); a small value exercises the fix-up path, a negative one makes every
 *                        wait give up at once (the fix-up launch then writes every tile).
 *   gmm_tile             128 forces the 128 x 128 GroupedMatmul kernel for every fp16/bf16 shape.
 */
void cb_set_test_overrides(int persistent_grid, int exchange_spin_limit, int gmm_tile);

/*
 * QuantMatmul (dense W8A8 with dequant epilogue).
 * Replaces quant_matmul(Tensor x1, Tensor x2, Tensor scale, *, Tensor? offset=None,
 *   Tensor? pertoken_scale=None, Tensor? bias=None, str? output_dtype=None) -> Tensor
 * (operators/quantmatmul/csrc/ops/quant_matmul/op_plugin/quant_matmul_plugin.cpp:48-49,77-267)
 * and qm_launch_cube_i32 + qm_launch_epilogue_{f16,bf16} (op_kernel/quant_matmul_launch.h:87-98).
 *
 *   x1 int8 [batch, M, K], x2 int8 [batch, K, N] (N contiguous), out [batch, M, N]
 *   scale      : scale_dtype (fp32 / bf16), scale_numel 1 or N
 *   offset     : fp32, offset_numel 0 (absent), 1 or N
 *   pertoken   : fp32, pertoken_numel 0 (absent) or M (indexed by row modulo M)
 *   bias       : bias_dtype (int32 / fp16 / bf16 / fp32), bias_numel 0 (absent), 1 or N,
 *                or batch*N when bias_batched != 0 (a [batch, 1, N] bias)
 *   out_dtype  : CB_DT_FLOAT16 (the reference's default) or CB_DT_BFLOAT16
 *   out[b,m,n] = cast((float(c) (+ i32 bias)) * scale (+ offset) (* pertoken[m]) (+ float bias))
 */
int cb_quant_matmul(const int8_t* x1, const int8_t* x2, const void* scale, int scale_dtype,
                    int64_t scale_numel, const float* offset, int64_t offset_numel,
                    const float* pertoken, int64_t pertoken_numel, const void* bias, int bias_dtype,
                    int64_t bias_numel, int bias_batched, int64_t batch, int64_t M, int64_t K,
                    int64_t N, int out_dtype, void* out, void* stream);

/*
 * int8 grouped down-projection (W8A8 GroupedMatmul with a per-token x per-channel dequant to bf16).
 * The reference has no int8 grouped matmul: the group semantics follow
 * grouped_matmul(Tensor x, Tensor weight, int[] group_list, ...) with split_item = 2 (one joined
 * output) (operators/groupedmatmul/csrc/ops/grouped_matmul/op_plugin/grouped_matmul_plugin.cpp:42-43,82-95)
 * and the epilogue follows QuantMatmul's scale-then-pertoken order
 * (operators/quantmatmul/csrc/ops/quant_matmul/op_kernel/quant_matmul_epilogue_kernel.cpp:273-292).
 *
 *   x int8 [M, K], weight int8 [E, K, N], weight_scale fp32 [E, N], x_scale fp32 [M]
 *   out bf16 [M, N]:  out[i, n] = bf16((float(x[i] . weight[g(i)][:, n]) * weight_scale[g, n]) * x_scale[i])
 */
int cb_grouped_matmul_quant(const int8_t* x, const int8_t* weight, const float* weight_scale,
                            const float* x_scale, const int64_t* group_list, int64_t group_len,
                            int64_t M, int64_t K, int64_t N, int64_t E, void* out, void* stream);

/*
 * GroupedMatmul, the float grouped GEMM: y[rows_g, :] = x[rows_g, :] @ weight[g] (+ bias[g, :]).
 * Replaces launch_gmm(x, w, b, y, ws, M, N, K, GmmGroupArg, xDtype, biasDtype, hasBias, transB,
 * stream) (operators/groupedmatmul/csrc/ops/grouped_matmul/op_kernel/grouped_matmul_launch.h:66-70)
 * with the plugin's checks (op_plugin/grouped_matmul_plugin.cpp:127-157) as status codes; no
 * workspace.  x_dtype and bias_dtype are CB_DT_FLOAT16 / CB_DT_BFLOAT16 / CB_DT_FLOAT32 (bias may be
 * NULL); at most 64 experts (GMM_MAX_E).
 *   x [M, K], weight [E, K, N] (transpose_weight = 0) or [E, N, K] (1), bias [E, N], y [M, N] in x_dtype
 * Accumulation in fp32, the bias added in fp32, one round-to-nearest-even narrowing.  K = 0 writes
 * the bias (or zeros).
 */
int cb_grouped_matmul(const void* x, const void* weight, const void* bias, int x_dtype, int bias_dtype,
                      const int64_t* group_list, int64_t group_len, int64_t M, int64_t K, int64_t N,
                      int64_t E, int transpose_weight, void* y, void* stream);

/*
 * Raw grouped int8 GEMM with exact int32 accumulation: c[rows_g, :] = x[rows_g, :] @ weight[g].
 * Replaces the reference's first GroupedMatmulSwigluQuant stage launch_gmsq_cube(x, w, c, ws, M, K,
 * N, E, GmsqGroupArg, stream) (op_kernel/gmsq_launch.h:67-69, gmsq_cube_kernel.cpp:15-16), which
 * writes the int32 [M, N] workspace its vector stage consumes.  Uses the same kernels as the fused
 * operators, with an int32 store epilogue.
 *   x int8 [M, K], weight int8 [E, K, N], c int32 [M, N]
 */
int cb_grouped_matmul_int32(const int8_t* x, const int8_t* weight, const int64_t* group_list,
                            int64_t group_len, int64_t M, int64_t K, int64_t N, int64_t E, int32_t* c,
                            void* stream);

/* ----------------------------------------------------------------------------------------------
 * Routing operators on either side of the expert FFN.
 * ---------------------------------------------------------------------------------------------- */

/* Workspace bytes cb_moe_re_routing needs for an [n_ranks, n_experts] count matrix. */
int64_t cb_moe_re_routing_workspace_size(int64_t n_ranks, int64_t n_experts);

/*
 * MoeReRouting: permute tokens received from n_ranks ranks (rank-major, each rank's block expert
 * ordered) into expert-major order.  Replaces moe_re_routing(tokens, expert_token_num_per_rank,
 * per_token_scales, expert_token_num_type, idx_type)
 * (operators/moererouting/csrc/ops/moe_re_routing/op_plugin/moe_re_routing_plugin.cpp:35-38,
 *  semantics op_kernel/moe_re_routing_kernel.cpp:15-24; only idx_type 0 exists there).
 *   tokens [A, H] (CB_DT_FLOAT16 / CB_DT_BFLOAT16 / CB_DT_INT8), counts [n_ranks, n_experts]
 *   (CB_DT_INT32 / CB_DT_INT64), per_token_scales fp32 [A] or NULL.
 *   Outputs: permute_tokens [A, H], permute_scales fp32 [A] (0 without scales), permute_idx int32 [A]
 *   (source row of each output row), expert_token_num [n_experts] (counts dtype; column sums).
 *   Rows past sum(counts) are left unwritten, as in the reference.  Any zero dimension returns CB_OK
 *   without writing (plugin :103-105).  n_ranks <= 1024.
 */
int cb_moe_re_routing(const void* tokens, int tokens_dtype, int64_t A, int64_t H, const void* counts,
                      int counts_dtype, int64_t n_ranks, int64_t n_experts, const float* per_token_scales,
                      void* permute_tokens, float* permute_scales, int32_t* permute_idx, void* expert_token_num,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * MoeFinalizeRouting: combine the K expert outputs of each token.  Replaces
 * moe_finalize_routing(expanded_permuted_rows, expanded_src_to_dst_row, skip1, skip2, bias, scales,
 * expert_for_source_row, drop_pad_mode)
 * (operators/moefinalizerouting/csrc/ops/moe_finalize_routing/op_plugin/moe_finalize_routing_plugin.cpp:33-36,
 *  semantics op_kernel/moe_finalize_routing_kernel.cpp:14-25):
 *   out[i, c] = skip1[i, c] + skip2[i, c] + sum_k scales[i, k] * (epr[p(i, k), c] + bias[eid(i, k), c])
 *   p(i, k) = esdr[k * num_rows + i] (drop_pad_mode 0/1) or esdr[i * K + k] (2/3); modes clamp to [0, 3];
 *   p outside [0, num_dst) drops the term; eid = expert_for_source_row[i * K + k] outside [0, n_bias_rows)
 *   drops only the bias.  Bias is used only together with expert_for_source_row.  fp32 accumulation in
 *   ascending k, round-half-even store.
 *   dtype: CB_DT_FLOAT16 / CB_DT_BFLOAT16 / CB_DT_FLOAT32 for epr, skips, bias and out; scales may be
 *   any of the three (scales_dtype) or NULL (then K is the caller's, normally 1).
 */
int cb_moe_finalize_routing(const void* expanded_permuted_rows, int dtype, int64_t num_dst, int64_t H,
                            const int32_t* expanded_src_to_dst_row, int64_t num_rows, int64_t K,
                            const void* skip1, const void* skip2, const void* bias, int64_t n_bias_rows,
                            const void* scales, int scales_dtype, const int32_t* expert_for_source_row,
                            int drop_pad_mode, void* out, void* stream);

/*
 * DequantSwigluQuant: dequant + SwiGLU + per-token int8 quantisation of an [M, 2H] row block.  Replaces
 * dequant_swiglu_quant(x, weight_scale, activation_scale, quant_scale, activate_left)
 * (operators/dequantswigluquant/csrc/ops/dequant_swiglu_quant/op_plugin/dqsq_plugin.cpp:34-35,
 *  operation order op_kernel/dqsq_kernel.cpp:334-427):
 *   A = x[:, :H], B = x[:, H:] as fp32; int32 x: A *= weight_scale[:H], B *= weight_scale[H:];
 *   quant_scale [H] multiplies the non-gate half; int32 x: A, B *= activation_scale[row];
 *   out = (A * B) / (1 + exp(-G)), G = B (activate_left 0) or A (activate_left 1);
 *   scale[row] = max(max|out| * (1/127), 1e-12); y = int8(rint(half(clamp(out / scale, -128, 127)))).
 *   x_dtype CB_DT_INT32 (weight_scale [2H] and activation_scale [M] required) or CB_DT_FLOAT16 /
 *   CB_DT_BFLOAT16 (both must be NULL).  y int8 [M, H], scale fp32 [M].
 */
int cb_dequant_swiglu_quant(const void* x, int x_dtype, int64_t M, int64_t N2, const float* weight_scale,
                            const float* activation_scale, const float* quant_scale, int activate_left,
                            int8_t* y, float* scale, void* stream);

/*
 * MoeGatingTopKSoftmax: fp32 softmax over the last dimension and its top k.  Replaces
 * moe_gating_top_k_softmax(x, finished, k)
 * (operators/moegatingtopksoftmax/csrc/ops/moe_gating_top_k_softmax/op_plugin/moe_gating_plugin.cpp:30,
 *  semantics op_kernel/moe_gating_kernel.cpp:15-21):
 *   y [rows, k] (x dtype) = the k largest softmax values in descending order (ties: lower column first);
 *   expert_idx int32 [rows, k] = their columns, or E for rows with finished[r] != 0;
 *   row_idx int32 [rows, k]: row_idx[r, j] = j * rows + r.
 *   x [rows, E] CB_DT_FLOAT32 / CB_DT_FLOAT16 / CB_DT_BFLOAT16, finished uint8/bool [rows] or NULL,
 *   0 < k <= E <= 2048.
 */
int cb_moe_gating_top_k_softmax(const void* x, int dtype, int64_t rows, int64_t E, const uint8_t* finished,
                                int64_t k, void* y, int32_t* expert_idx, int32_t* row_idx, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* CANNBENCH_AMD_H */
