/*
 * cb_oracle.c - CPU restatement of the reference operators' arithmetic.  TEST INFRASTRUCTURE ONLY.
 *
 * This file is the checker for the HIP library: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it.  The product path never calls it.
 *
 * It restates, from the reference kernels' documented semantics (not from their code), the
 * per-element arithmetic of every operator on the path, in plain C with OpenMP:
 *
 *   or_dynamic_quant   operators/dynamicquant/csrc/ops/dynamic_quant/op_kernel/dynamic_quant_kernel.cpp:15-26,240-282
 *   or_ardq            operators/addrmsnormdynamicquant/csrc/ops/add_rms_norm_dynamic_quant/op_kernel/
 *                      add_rms_norm_dynamic_quant_kernel.cpp:15-30,413-503
 *   or_i8_gemm         operators/groupedmatmulswigluquant/.../op_kernel/gmsq_cube_kernel.cpp:15-16 (exact int32)
 *   or_gmsq            operators/groupedmatmulswigluquant/.../op_kernel/gmsq_vec_kernel.cpp:15-20,184-264
 *                      with the group routing of op_plugin/gmsq_plugin.cpp:101-117
 *   or_quant_matmul    operators/quantmatmul/csrc/ops/quant_matmul/op_kernel/quant_matmul_epilogue_kernel.cpp:15-22,243-305
 *   or_grouped_matmul_quant  group routing of operators/groupedmatmul/.../op_plugin/grouped_matmul_plugin.cpp:82-95
 *                      with the QuantMatmul epilogue order (no reference op exists: parity unpinned by the
 *                      reference, pinned here only by the closed forms the tests check)
 *   or_grouped_matmul  operators/groupedmatmul/csrc/ops/grouped_matmul/op_plugin/grouped_matmul_plugin.cpp:14-17
 *                      and op_kernel/grouped_matmul_kernel.cpp:15-17,111-150 (float GEMM per expert + bias)
 *   or_moe_re_routing        operators/moererouting/.../op_kernel/moe_re_routing_kernel.cpp:15-24
 *   or_moe_finalize_routing  operators/moefinalizerouting/.../op_kernel/moe_finalize_routing_kernel.cpp:14-25,137-183
 *   or_dequant_swiglu_quant  operators/dequantswigluquant/.../op_kernel/dqsq_kernel.cpp:15-27,334-427,476-524
 *   or_moe_gating_top_k_softmax  operators/moegatingtopksoftmax/.../op_kernel/moe_gating_kernel.cpp:15-21,318-390
 *
 * Rounding conventions (all round-half-to-even):
 *   rint16(v)  fp32 -> fp16 -> int8, the reference's two-step narrowing (dynamic_quant_kernel.cpp:20-22,
 *              add_rms_norm_dynamic_quant_kernel.cpp:74-76, gmsq_vec_kernel.cpp:256-257).  NaN -> 0,
 *              out-of-range values saturate.
 *   bf16/fp16 outputs: fp32 -> 16-bit RNE.
 *
 * Pinning: tests/test_oracle.py checks each function against brute-force numpy on small inputs,
 * closed forms (exact int32 GEMM vs int64 matmul, E=1 reduction of GMSQ to QuantMatmul + SwiGLU +
 * DynamicQuant), invariants (|y| <= 127, max|y| in {126,127}, y*scale ~ input) and the golden
 * fixtures under tests/golden/.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DT_F16 1
#define DT_BF16 2
#define DT_F32 3
#define DT_I8 4
#define DT_I32 5

static const float FLT_MIN_F = 1.1754944e-38f;

static inline uint32_t f_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float bits_f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float or_bf16_to_f32(uint16_t h) { return bits_f(((uint32_t)h) << 16); }

uint16_t or_f32_to_bf16(float f)
{
    uint32_t u = f_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float or_f16_to_f32(uint16_t h)
{
    uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0) {
        /* zero / subnormal: m * 2^-24 is exact in fp32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return (s ? -v : v);
    }
    if (e == 31) return bits_f(s | 0x7f800000u | (m << 13));
    return bits_f(s | ((e + 112u) << 23) | (m << 13));
}

uint16_t or_f32_to_f16(float f)
{
    uint32_t u = f_bits(f);
    uint16_t s = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(s | 0x7e00u);      /* NaN */
    if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u);      /* >= 65520 rounds to inf */
    if (a < 0x38800000u) {
        /* below 2^-14: fp16 subnormal range, quantum 2^-24.  x * 2^24 is exact; rint is RNE. */
        float x = bits_f(a) * 16777216.0f;
        return (uint16_t)(s | (uint16_t)nearbyintf(x));
    }
    /* normal: drop 13 mantissa bits with RNE */
    uint32_t e = (a >> 23) - 112u;
    uint32_t m = a & 0x7fffffu;
    uint32_t h = (e << 10) | (m >> 13);
    uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u; /* carry may bump exponent: ok */
    return (uint16_t)(s | h);
}

/* fp32 -> fp16 (RNE) -> int8 (RNE, saturating, NaN -> 0). */
int8_t or_rint16(float v)
{
    float h = or_f16_to_f32(or_f32_to_f16(v));
    if (h != h) return 0;
    float r = nearbyintf(h);
    if (r > 127.0f) return 127;
    if (r < -128.0f) return -128;
    return (int8_t)r;
}

static inline float load16(const uint16_t* p, int64_t i, int dtype)
{
    return dtype == DT_BF16 ? or_bf16_to_f32(p[i]) : or_f16_to_f32(p[i]);
}

static inline uint16_t store16(float v, int dtype)
{
    return dtype == DT_BF16 ? or_f32_to_bf16(v) : or_f32_to_f16(v);
}

/* DynamicQuant, one row at a time (dynamic_quant_kernel.cpp:15-26):
 *   a = max(max_j |x_j|, 1e-12); scale = a * (1/127); y = rint16(x * (127 * (1/a))). */
void or_dynamic_quant(const uint16_t* x, int dtype, int64_t rows, int64_t n, int8_t* y, float* scale)
{
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* xr = x + r * n;
        float a = 0.0f;
        for (int64_t j = 0; j < n; ++j) {
            float v = fabsf(load16(xr, j, dtype));
            if (v > a) a = v; /* NaN elements never win the max */
        }
        if (a < 1e-12f) a = 1e-12f;
        scale[r] = a * (1.0f / 127.0f);
        float inv = 127.0f * (1.0f / a);
        for (int64_t j = 0; j < n; ++j) y[r * n + j] = or_rint16(load16(xr, j, dtype) * inv);
    }
}

/* AddRmsNormDynamicQuant (add_rms_norm_dynamic_quant_kernel.cpp:15-30, 440-497):
 *   xf = x1 + x2 (fp32); xOut = round16(xf); ss = sum xf^2 (of the unrounded sum);
 *   rstd = 1 / sqrt(ss * (1/n) + eps); z = xf * gamma; m = max|z| * rstd;
 *   scale = max(m, 1e-12) * (1/127); k = rstd / scale; y = rint16(z * k).
 * The sum of squares is accumulated in double and rounded once (the reference adds in fp32 lanes;
 * the two differ by a few ulp, inside the stated tolerance). */
void or_ardq(const uint16_t* x1, const uint16_t* x2, const uint16_t* gamma, int dtype, int64_t rows,
             int64_t n, float eps, int8_t* y, uint16_t* xout, float* scale)
{
    const float invN = 1.0f / (float)n;
#pragma omp parallel
    {
        float* z = (float*)malloc(sizeof(float) * (size_t)n);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            double ss = 0.0;
            float mz = 0.0f;
            int nan = 0;
            for (int64_t j = 0; j < n; ++j) {
                float xf = load16(x1, r * n + j, dtype) + load16(x2, r * n + j, dtype);
                xout[r * n + j] = store16(xf, dtype);
                ss += (double)xf * (double)xf;
                z[j] = xf * load16(gamma, j, dtype);
                float az = fabsf(z[j]);
                if (az != az) nan = 1;
                if (az > mz) mz = az;
            }
            if (nan) mz = NAN;
            float rms = sqrtf((float)ss * invN + eps);
            float rstd = 1.0f / rms;
            float m = mz * rstd;
            float sm = (m < 1e-12f) ? 1e-12f : m;
            float sc = sm * (1.0f / 127.0f);
            float k = rstd / sc;
            scale[r] = sc;
            for (int64_t j = 0; j < n; ++j) y[r * n + j] = or_rint16(z[j] * k);
        }
        free(z);
    }
}

/* Exact int8 x int8 -> int32 GEMM: c[i, j] = sum_k a[i, k] * b[k, j] for i in [0, m).
 * a row stride lda, b row stride ldb (N contiguous), c row stride ldc.  |c| <= 127*128*K. */
void or_i8_gemm(const int8_t* a, int64_t lda, const int8_t* b, int64_t ldb, int32_t* c, int64_t ldc,
                int64_t m, int64_t k, int64_t n)
{
    const int64_t CJ = 512;
    int64_t nchunks = (n + CJ - 1) / CJ;
    int64_t rblocks = (m + 3) / 4;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int64_t rb = 0; rb < rblocks; ++rb) {
        for (int64_t jc = 0; jc < nchunks; ++jc) {
            int64_t j0 = jc * CJ, j1 = j0 + CJ < n ? j0 + CJ : n, w = j1 - j0;
            int64_t r0 = rb * 4, r1 = r0 + 4 < m ? r0 + 4 : m;
            int32_t acc[4][512];
            memset(acc, 0, sizeof(acc));
            for (int64_t kk = 0; kk < k; ++kk) {
                const int8_t* br = b + kk * ldb + j0;
                for (int64_t r = r0; r < r1; ++r) {
                    int32_t av = a[r * lda + kk];
                    int32_t* ar = acc[r - r0];
                    for (int64_t j = 0; j < w; ++j) ar[j] += av * (int32_t)br[j];
                }
            }
            for (int64_t r = r0; r < r1; ++r)
                memcpy(c + r * ldc + j0, acc[r - r0], sizeof(int32_t) * (size_t)w);
        }
    }
}

/* Group of a row from the cumsum group_list: the g with gl[g-1] <= row < gl[g]. */
static int64_t group_of(const int64_t* gl, int64_t E, int64_t row)
{
    int64_t lo = 0, hi = E - 1;
    while (lo < hi) {
        int64_t mid = (lo + hi) / 2;
        if (gl[mid] > row) hi = mid; else lo = mid + 1;
    }
    return lo;
}

/* Reference SwiGLU epilogue for one row (gmsq_vec_kernel.cpp:15-20, 207-257). */
static void gmsq_row_epilogue(const int32_t* c, float xs, const float* ws, int64_t N, int8_t* y,
                              float* ys, float* act)
{
    const int64_t H = N / 2;
    float amax = 0.0f;
    for (int64_t j = 0; j < H; ++j) {
        float L = ((float)c[j] * xs) * ws[j];
        float R = ((float)c[j + H] * xs) * ws[j + H];
        float a = (L / (1.0f + expf(-L))) * R;
        act[j] = a;
        float aa = fabsf(a);
        if (aa > amax) amax = aa;
    }
    if (!(amax > FLT_MIN_F)) amax = FLT_MIN_F;
    *ys = amax * (1.0f / 127.0f);
    /* The reference clamps to [-128, 127] before narrowing (gmsq_vec_kernel.cpp:253-257); the
     * saturating rint16 gives the same result for every non-NaN value.  For an all-zero row
     * 127 / FLT_MIN overflows to inf and 0 * inf is NaN, which narrows to 0 (y = round(0 / scale)). */
    float inv = 127.0f / amax;
    for (int64_t j = 0; j < H; ++j) y[j] = or_rint16(act[j] * inv);
}

/* GroupedMatmulSwigluQuant for rows [row_begin, row_end) (all rows when row_end <= row_begin is
 * not the case; callers pass 0, M for the full op).  y is [M, N/2] and y_scale [M]; only the
 * requested rows are written. */
void or_gmsq(const int8_t* x, const int8_t* w, const float* ws, const float* xs, const int64_t* gl,
             int64_t E, int64_t M, int64_t K, int64_t N, int64_t row_begin, int64_t row_end,
             int8_t* y, float* ys)
{
    (void)M;
    const int64_t H = N / 2;
    int64_t r = row_begin;
    int32_t* c = NULL;
    float* act = (float*)malloc(sizeof(float) * (size_t)H);
    while (r < row_end) {
        int64_t g = group_of(gl, E, r);
        int64_t gend = gl[g] < row_end ? gl[g] : row_end;
        int64_t nr = gend - r;
        c = (int32_t*)realloc(c, sizeof(int32_t) * (size_t)(nr * N));
        or_i8_gemm(x + r * K, K, w + g * K * N, N, c, N, nr, K, N);
        for (int64_t i = 0; i < nr; ++i)
            gmsq_row_epilogue(c + i * N, xs[r + i], ws + g * N, N, y + (r + i) * H, ys + r + i, act);
        r = gend;
    }
    free(act);
    free(c);
}

/* QuantMatmul epilogue chain (quant_matmul_epilogue_kernel.cpp:15-22, 261-305) for rows
 * [row_begin, row_end) of every batch.  Flags describe which optional inputs are present. */
static float load_any(const void* p, int dtype, int64_t i)
{
    switch (dtype) {
    case DT_F16: return or_f16_to_f32(((const uint16_t*)p)[i]);
    case DT_BF16: return or_bf16_to_f32(((const uint16_t*)p)[i]);
    case DT_I32: return (float)((const int32_t*)p)[i];
    default: return ((const float*)p)[i];
    }
}

void or_quant_matmul(const int8_t* x1, const int8_t* x2, const void* scale, int scale_dtype,
                     int64_t scale_numel, const float* offset, int64_t offset_numel,
                     const float* pertoken, int64_t pertoken_numel, const void* bias, int bias_dtype,
                     int64_t bias_numel, int bias_batched, int64_t batch, int64_t M, int64_t K,
                     int64_t N, int out_dtype, uint16_t* out, int64_t row_begin, int64_t row_end)
{
    int64_t nr = row_end - row_begin;
    if (nr <= 0) return;
    int32_t* c = (int32_t*)malloc(sizeof(int32_t) * (size_t)(nr * N));
    for (int64_t b = 0; b < batch; ++b) {
        or_i8_gemm(x1 + (b * M + row_begin) * K, K, x2 + b * K * N, N, c, N, nr, K, N);
        const int64_t boff = bias_batched ? b * N : 0;
#pragma omp parallel for schedule(static)
        for (int64_t i = 0; i < nr; ++i) {
            int64_t m = row_begin + i;
            for (int64_t n = 0; n < N; ++n) {
                float v = (float)c[i * N + n];
                if (bias_numel > 0 && bias_dtype == DT_I32)
                    v = v + load_any(bias, bias_dtype, boff + (bias_numel == 1 ? 0 : n));
                v = v * load_any(scale, scale_dtype, scale_numel == 1 ? 0 : n);
                if (offset_numel > 0) v = v + offset[offset_numel == 1 ? 0 : n];
                if (pertoken_numel > 0) v = v * pertoken[m];
                if (bias_numel > 0 && bias_dtype != DT_I32)
                    v = v + load_any(bias, bias_dtype, boff + (bias_numel == 1 ? 0 : n));
                out[(b * M + m) * N + n] = store16(v, out_dtype);
            }
        }
    }
    free(c);
}

/* int8 grouped down-projection for rows [row_begin, row_end):
 *   out[i, n] = bf16((float(c[i, n]) * ws[g, n]) * xs[i]). */
void or_grouped_matmul_quant(const int8_t* x, const int8_t* w, const float* ws, const float* xs,
                             const int64_t* gl, int64_t E, int64_t M, int64_t K, int64_t N,
                             int64_t row_begin, int64_t row_end, uint16_t* out)
{
    (void)M;
    int64_t r = row_begin;
    int32_t* c = NULL;
    while (r < row_end) {
        int64_t g = group_of(gl, E, r);
        int64_t gend = gl[g] < row_end ? gl[g] : row_end;
        int64_t nr = gend - r;
        c = (int32_t*)realloc(c, sizeof(int32_t) * (size_t)(nr * N));
        or_i8_gemm(x + r * K, K, w + g * K * N, N, c, N, nr, K, N);
        for (int64_t i = 0; i < nr; ++i)
            for (int64_t n = 0; n < N; ++n)
                out[(r + i) * N + n] =
                    or_f32_to_bf16(((float)c[i * N + n] * ws[g * N + n]) * xs[r + i]);
        r = gend;
    }
    free(c);
}

/* ============================================================================================
 * Routing operators on either side of the expert FFN.
 * ============================================================================================ */

/* GroupedMatmul (grouped_matmul_plugin.cpp:14-17, grouped_matmul_kernel.cpp:111-150): for the rows
 * of expert g, y = x @ w[g] (+ bias[g]).  The reference accumulates on its matrix unit in fp32 in an
 * order of its own; this restatement accumulates in double (the exact sum up to double rounding),
 * adds the bias in double, then narrows double -> fp32 -> the output dtype (RNE), so a GPU result
 * within the fp32 accumulation error of the exact sum agrees to one output ulp.
 * Elements: fp16 / bf16 as uint16 bits, fp32 as float; w [E, K, N] or, with trans, [E, N, K]. */
static inline double gload(const void* p, int dt, int64_t i)
{
    if (dt == DT_F32) return (double)((const float*)p)[i];
    return (double)load16((const uint16_t*)p, i, dt);
}

void or_grouped_matmul(const void* x, const void* w, const void* bias, int x_dt, int bias_dt, const int64_t* gl,
                       int64_t E, int64_t M, int64_t K, int64_t N, int trans, void* y)
{
    (void)M; /* the rows are gl[E - 1] == M */
    for (int64_t g = 0; g < E; ++g) {
        const int64_t r0 = g ? gl[g - 1] : 0, r1 = gl[g];
        const int64_t wb = g * K * N;
#pragma omp parallel for schedule(static)
        for (int64_t r = r0; r < r1; ++r) {
            for (int64_t n = 0; n < N; ++n) {
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k)
                    acc += gload(x, x_dt, r * K + k) * gload(w, x_dt, wb + (trans ? n * K + k : k * N + n));
                if (bias) acc += gload(bias, bias_dt, g * N + n);
                const float f = (float)acc;
                if (x_dt == DT_F32) ((float*)y)[r * N + n] = f;
                else ((uint16_t*)y)[r * N + n] = store16(f, x_dt);
            }
        }
    }
}

/* MoeReRouting (operators/moererouting/csrc/ops/moe_re_routing/op_kernel/moe_re_routing_kernel.cpp:15-24):
 * the (rank i, expert j) cell's cnt[i][j] rows move from source offset
 * rowStart(i) + sum_{j'<j} cnt[i][j'] to destination offset colStart(j) + sum_{i'<i} cnt[i'][j].
 * Written as the direct double loop over cells, in the order of that definition.
 * counts are int64 here (the wrapper widens int32).  Returns the routed total. */
int64_t or_moe_re_routing(const uint8_t* tokens, int64_t A, int64_t row_bytes, const int64_t* cnt,
                          int64_t n, int64_t e, const float* scales, uint8_t* out_tok, float* out_sc,
                          int32_t* out_idx, int64_t* etn)
{
    int64_t* dst = (int64_t*)malloc(sizeof(int64_t) * (size_t)(e > 0 ? e : 1));
    int64_t run = 0;
    for (int64_t j = 0; j < e; ++j) {
        int64_t col = 0;
        for (int64_t i = 0; i < n; ++i) col += cnt[i * e + j];
        etn[j] = col;
        dst[j] = run; /* colStart(j), advanced by each rank's count below */
        run += col;
    }
    int64_t src = 0; /* rowStart(i) + sum_{j'<j} cnt[i][j'] */
    for (int64_t i = 0; i < n; ++i) {
        for (int64_t j = 0; j < e; ++j) {
            const int64_t c = cnt[i * e + j];
            for (int64_t k = 0; k < c; ++k) {
                const int64_t s = src + k, d = dst[j] + k;
                if (s < 0 || s >= A || d < 0 || d >= A) continue;
                memcpy(out_tok + d * row_bytes, tokens + s * row_bytes, (size_t)row_bytes);
                out_sc[d] = scales ? scales[s] : 0.0f;
                out_idx[d] = (int32_t)s;
            }
            src += c;
            dst[j] += c;
        }
    }
    free(dst);
    return run;
}

/* MoeFinalizeRouting (operators/moefinalizerouting/csrc/ops/moe_finalize_routing/op_kernel/
 * moe_finalize_routing_kernel.cpp:14-25, 137-183): fp32 accumulation, ascending k, RNE store.
 * Null skip / bias / scales / expert pointers mean absent. */
void or_moe_finalize_routing(const void* epr, int dtype, int64_t num_dst, int64_t H, const int32_t* esdr,
                             int64_t num_rows, int64_t K, const void* skip1, const void* skip2,
                             const void* bias, int64_t n_bias, const void* scales, int scales_dtype,
                             const int32_t* expert, int mode, void* out)
{
    if (mode < 0) mode = 0;
    if (mode > 3) mode = 3;
    if (!expert) bias = NULL;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < num_rows; ++i) {
        for (int64_t c = 0; c < H; ++c) {
            float acc = 0.0f;
            if (skip1) acc = load_any(skip1, dtype, i * H + c);
            if (skip2) acc = acc + load_any(skip2, dtype, i * H + c);
            for (int64_t k = 0; k < K; ++k) {
                const int64_t p = esdr[mode <= 1 ? k * num_rows + i : i * K + k];
                if (p < 0 || p >= num_dst) continue;
                float term = load_any(epr, dtype, p * H + c);
                if (bias) {
                    const int64_t eid = expert[i * K + k];
                    if (eid >= 0 && eid < n_bias) term = term + load_any(bias, dtype, eid * H + c);
                }
                if (scales) term = term * load_any(scales, scales_dtype, i * K + k);
                acc = acc + term;
            }
            if (dtype == DT_F32) ((float*)out)[i * H + c] = acc;
            else ((uint16_t*)out)[i * H + c] = store16(acc, dtype);
        }
    }
}

/* DequantSwigluQuant (operators/dequantswigluquant/csrc/ops/dequant_swiglu_quant/op_kernel/
 * dqsq_kernel.cpp:15-27, 334-427, 476-524).  x is int32 / fp16 / bf16 [M, 2H]. */
void or_dequant_swiglu_quant(const void* x, int x_dtype, int64_t M, int64_t H, const float* ws,
                             const float* as, const float* qs, int act_left, int8_t* y, float* scale)
{
#pragma omp parallel
    {
        float* out = (float*)malloc(sizeof(float) * (size_t)(H > 0 ? H : 1));
#pragma omp for schedule(static)
        for (int64_t r = 0; r < M; ++r) {
            float amax = 0.0f;
            for (int64_t j = 0; j < H; ++j) {
                float A = load_any(x, x_dtype, r * 2 * H + j), B = load_any(x, x_dtype, r * 2 * H + H + j);
                if (x_dtype == DT_I32) {
                    A = A * ws[j];
                    B = B * ws[H + j];
                }
                if (qs) {
                    if (act_left) B = B * qs[j];
                    else A = A * qs[j];
                }
                if (x_dtype == DT_I32) {
                    A = A * as[r];
                    B = B * as[r];
                }
                const float G = act_left ? A : B;
                out[j] = (A * B) / (1.0f + expf(-G));
                const float a = fabsf(out[j]);
                if (a > amax) amax = a;
            }
            float s = amax * (1.0f / 127.0f);
            if (!(s >= 1e-12f)) s = 1e-12f;
            scale[r] = s;
            for (int64_t j = 0; j < H; ++j) {
                float q = out[j] / s;
                q = q > 127.0f ? 127.0f : (q < -128.0f ? -128.0f : q);
                y[r * H + j] = or_rint16(q);
            }
        }
        free(out);
    }
}

/* MoeGatingTopKSoftmax (operators/moegatingtopksoftmax/csrc/ops/moe_gating_top_k_softmax/op_kernel/
 * moe_gating_kernel.cpp:15-21, 318-390): e = exp(x - max) in fp32, sum = sum(e); the k largest e in
 * descending order (equal values: lower column first, the order of a stable sort), y = e / sum narrowed
 * RNE to the x dtype; expert_idx = column (E for finished rows); row_idx = j * rows + r.
 * Selection is k passes of a linear arg-max scan, so it is a brute-force restatement of the sort. */
void or_moe_gating_top_k_softmax(const void* x, int dtype, int64_t rows, int64_t E, const uint8_t* finished,
                                 int64_t k, void* y, int32_t* eidx, int32_t* ridx)
{
#pragma omp parallel
    {
        float* e = (float*)malloc(sizeof(float) * (size_t)E);
        uint8_t* used = (uint8_t*)malloc((size_t)E);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            float m = -INFINITY;
            for (int64_t c = 0; c < E; ++c) {
                e[c] = load_any(x, dtype, r * E + c);
                if (e[c] > m) m = e[c];
            }
            float s = 0.0f;
            for (int64_t c = 0; c < E; ++c) {
                e[c] = expf(e[c] - m);
                used[c] = 0;
            }
            for (int64_t c = 0; c < E; ++c) s += e[c];
            for (int64_t j = 0; j < k; ++j) {
                int64_t b = -1;
                for (int64_t c = 0; c < E; ++c)
                    if (!used[c] && (b < 0 || e[c] > e[b])) b = c;
                used[b] = 1;
                const float v = e[b] / s;
                if (dtype == DT_F32) ((float*)y)[r * k + j] = v;
                else ((uint16_t*)y)[r * k + j] = store16(v, dtype);
                eidx[r * k + j] = (finished && finished[r]) ? (int32_t)E : (int32_t)b;
                ridx[r * k + j] = (int32_t)(j * rows + r);
            }
        }
        free(e);
        free(used);
    }
}
