// moe_routing.hip - the operators on either side of the MoE-FFN path, for gfx950:
//   cb_moe_re_routing            token permutation rank-major -> expert-major (feeds GMSQ)
//   cb_moe_finalize_routing      weighted combine of expert outputs + skips + bias (after the
//                                down-projection)
//   cb_dequant_swiglu_quant      standalone dequant + SwiGLU + per-token int8 quant
//   cb_moe_gating_top_k_softmax  softmax + top-k routing producer
// All four are HBM-bound gather / row kernels: rows are moved with 16-byte accesses, per-row
// reductions are wave / workgroup shuffles, and nothing is staged through host memory.
#include <cstring>

#include "common.hpp"
#include "host_util.hpp"

namespace cb {

typedef int iv4 __attribute__((ext_vector_type(4)));

// ============================================================================================
// MoeReRouting
//   Reference semantics (operators/moererouting/csrc/ops/moe_re_routing/op_kernel/
//   moe_re_routing_kernel.cpp:15-24):
//     srcStart(i,j) = rowStart(i) + sum_{j'<j} cnt[i][j']
//     dstStart(i,j) = colStart(j) + sum_{i'<i} cnt[i'][j]
//     permute_tokens[dstStart+k] = tokens[srcStart+k]; permute_scales likewise (0 without
//     scales); permute_idx[dstStart+k] = srcStart+k; expert_token_num[j] = sum_i cnt[i][j]
// ============================================================================================
struct RerouteWs {
    int64_t src_off, dst_off, col_off, total;
};

static RerouteWs reroute_ws(int64_t n, int64_t e)
{
    RerouteWs w;
    auto up = [](int64_t v) { return (v + 255) / 256 * 256; };
    w.src_off = 0;
    w.dst_off = up(n * e * 4);
    w.col_off = w.dst_off + up(n * e * 4);
    w.total = w.col_off + up((e + 1) * 4);
    return w;
}

template <typename CT>
__global__ __launch_bounds__(1024) void mrr_prefix_kernel(const CT* __restrict__ cnt, int n, int e,
                                                          int32_t* __restrict__ src_start,
                                                          int32_t* __restrict__ dst_start,
                                                          int32_t* __restrict__ col_start, CT* __restrict__ etn)
{
    __shared__ int64_t sh[1024];
    const int t = threadIdx.x;
    // rows: exclusive prefix along experts -> src_start relative to the row start; row totals in sh
    for (int i = t; i < n; i += blockDim.x) {
        int64_t run = 0;
        for (int j = 0; j < e; ++j) {
            src_start[(int64_t)i * e + j] = (int32_t)run;
            run += (int64_t)cnt[(int64_t)i * e + j];
        }
    }
    __syncthreads();
    // row starts: exclusive scan of the row totals, serial (n is the rank count)
    if (t == 0) {
        int64_t run = 0;
        for (int i = 0; i < n; ++i) {
            const int64_t last = (int64_t)src_start[(int64_t)i * e + e - 1] + (int64_t)cnt[(int64_t)i * e + e - 1];
            sh[i % 1024] = run;  // only used when n <= 1024 (checked on the host)
            run += last;
        }
    }
    __syncthreads();
    for (int i = t; i < n; i += blockDim.x) {
        const int64_t rs = sh[i];
        for (int j = 0; j < e; ++j) src_start[(int64_t)i * e + j] += (int32_t)rs;
    }
    // columns: totals (expert_token_num) and exclusive prefix along ranks
    for (int j = t; j < e; j += blockDim.x) {
        int64_t run = 0;
        for (int i = 0; i < n; ++i) {
            dst_start[(int64_t)i * e + j] = (int32_t)run;
            run += (int64_t)cnt[(int64_t)i * e + j];
        }
        etn[j] = (CT)run;
    }
    __syncthreads();
    if (t == 0) {
        int64_t run = 0;
        for (int j = 0; j < e; ++j) {
            col_start[j] = (int32_t)run;
            run += (int64_t)etn[j];
        }
        col_start[e] = (int32_t)run;
    }
    __syncthreads();
    for (int j = t; j < e; j += blockDim.x) {
        const int32_t cs = col_start[j];
        for (int i = 0; i < n; ++i) dst_start[(int64_t)i * e + j] += cs;
    }
}

// One wave per destination row: locate the (rank, expert) cell, then copy the row.
__global__ __launch_bounds__(256) void mrr_gather_kernel(const uint8_t* __restrict__ tokens, int64_t a,
                                                         int64_t row_bytes, const float* __restrict__ scales,
                                                         const int32_t* __restrict__ src_start,
                                                         const int32_t* __restrict__ dst_start,
                                                         const int32_t* __restrict__ col_start, int n, int e,
                                                         uint8_t* __restrict__ out_tok, float* __restrict__ out_sc,
                                                         int32_t* __restrict__ out_idx, int vec16)
{
    const int lane = threadIdx.x & 63;
    const int64_t d = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t total = col_start[e];
    if (d >= a || d >= total) return;  // rows past the routed total are not written (as the reference)
    // expert j: last column with col_start[j] <= d
    int lo = 0, hi = e - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (col_start[mid] <= d) lo = mid;
        else hi = mid - 1;
    }
    const int j = lo;
    // rank i: last rank with dst_start[i][j] <= d
    int ilo = 0, ihi = n - 1;
    while (ilo < ihi) {
        const int mid = (ilo + ihi + 1) >> 1;
        if (dst_start[(int64_t)mid * e + j] <= d) ilo = mid;
        else ihi = mid - 1;
    }
    const int64_t src = (int64_t)src_start[(int64_t)ilo * e + j] + (d - dst_start[(int64_t)ilo * e + j]);
    if (src < 0 || src >= a) return;
    if (lane == 0) {
        out_sc[d] = scales ? scales[src] : 0.0f;
        out_idx[d] = (int32_t)src;
    }
    const uint8_t* s = tokens + src * row_bytes;
    uint8_t* o = out_tok + d * row_bytes;
    if (vec16) {
        const int64_t nv = row_bytes >> 4;
        for (int64_t v = lane; v < nv; v += 64)
            __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const iv4*>(s) + v),
                                        reinterpret_cast<iv4*>(o) + v);
    } else {
        for (int64_t b = lane; b < row_bytes; b += 64) o[b] = s[b];
    }
}

// ============================================================================================
// MoeFinalizeRouting
//   Reference semantics (operators/moefinalizerouting/csrc/ops/moe_finalize_routing/op_kernel/
//   moe_finalize_routing_kernel.cpp:15-25, 132-183, 230-245):
//     acc = f32(skip1) [+ f32(skip2)]              (0 without skips)
//     for k ascending: p = esdr[k*R + i] (modes 0/1) or esdr[i*K + k] (modes 2/3); p outside
//       [0, numDst) -> no term; term = f32(epr[p]) [+ f32(bias[eid])] if bias and 0 <= eid < E;
//       term *= f32(scales[i, k]) when scales are given; acc += term
//     out = round-half-even(acc) to the row dtype
// ============================================================================================
template <int DT>
__device__ __forceinline__ float ld_any(const void* p, int64_t i)
{
    if constexpr (DT == CB_DT_FLOAT32) return ((const float*)p)[i];
    else if constexpr (DT == CB_DT_BFLOAT16) return bf16_to_f32(((const uint16_t*)p)[i]);
    else return f16_to_f32(((const uint16_t*)p)[i]);
}

template <int DT>
__device__ __forceinline__ void st_any(void* p, int64_t i, float v)
{
    if constexpr (DT == CB_DT_FLOAT32) ((float*)p)[i] = v;
    else if constexpr (DT == CB_DT_BFLOAT16) ((uint16_t*)p)[i] = f32_to_bf16(v);
    else ((uint16_t*)p)[i] = f32_to_f16(v);
}

struct MfrArgs {
    const void* epr;
    const int32_t* esdr;
    const void* skip1;
    const void* skip2;
    const void* bias;
    const void* scales;
    const int32_t* expert;
    void* out;
    int64_t num_dst, num_rows, H, K, E;
    int32_t col_mode, scales_dt;
};

template <int DT, int SDT>
__global__ __launch_bounds__(256) void mfr_kernel(const MfrArgs a)
{
    const int64_t i = blockIdx.x;
    const int64_t H = a.H, K = a.K;
    const int64_t row = i * H;
    // one pass over the row: each thread owns columns t, t + 256, ...
    for (int64_t c = threadIdx.x; c < H; c += blockDim.x) {
        float acc = 0.0f;
        if (a.skip1) acc = ld_any<DT>(a.skip1, row + c);
        if (a.skip2) acc = acc + ld_any<DT>(a.skip2, row + c);
        for (int64_t k = 0; k < K; ++k) {
            const int64_t p = a.esdr[a.col_mode ? k * a.num_rows + i : i * K + k];
            if (p < 0 || p >= a.num_dst) continue;
            float term = ld_any<DT>(a.epr, p * H + c);
            if (a.bias) {
                const int64_t eid = a.expert[i * K + k];
                if (eid >= 0 && eid < a.E) term = term + ld_any<DT>(a.bias, eid * H + c);
            }
            if (a.scales) term = term * ld_any<SDT>(a.scales, i * K + k);
            acc = acc + term;
        }
        st_any<DT>(a.out, row + c, acc);
    }
}

// ============================================================================================
// DequantSwigluQuant
//   Reference semantics (operators/dequantswigluquant/csrc/ops/dequant_swiglu_quant/op_kernel/
//   dqsq_kernel.cpp:15-27 and the operation order of :336-427, 476-524):
//     A = f32(x[:, :H]) [* weight_scale[:H]], B = f32(x[:, H:]) [* weight_scale[H:]]   (int32 x)
//     the non-gate half *= quant_scale                     (when given)
//     A *= activation_scale[row], B *= activation_scale[row] (int32 x)
//     out = (A * B) / (1 + exp(-G)),  G = B (activate_left false) or A (true)
//     s = max(max_j |out| * (1/127), 1e-12);  y = rint16(clamp(out / s, -128, 127))
// ============================================================================================
template <int XDT>
__device__ __forceinline__ float ld_x(const void* x, int64_t i)
{
    if constexpr (XDT == CB_DT_INT32) return (float)((const int32_t*)x)[i];
    else if constexpr (XDT == CB_DT_BFLOAT16) return bf16_to_f32(((const uint16_t*)x)[i]);
    else return f16_to_f32(((const uint16_t*)x)[i]);
}

constexpr int kDqsqMaxPerThread = 16;

template <int XDT>
__device__ __forceinline__ float dqsq_elem(const void* x, int64_t base, int64_t H, int64_t j, const float* ws,
                                           float asr, const float* qs, int act_left)
{
    float A = ld_x<XDT>(x, base + j), B = ld_x<XDT>(x, base + H + j);
    if constexpr (XDT == CB_DT_INT32) {
        A = A * ws[j];
        B = B * ws[H + j];
    }
    if (qs) {
        if (act_left) B = B * qs[j];
        else A = A * qs[j];
    }
    if constexpr (XDT == CB_DT_INT32) {
        A = A * asr;
        B = B * asr;
    }
    const float G = act_left ? A : B;
    return (A * B) / (1.0f + expf(-G));
}

// REG: the row's results stay in registers between the max and the quantisation (H <= 16 * blockDim);
// otherwise the second pass recomputes them (identical arithmetic, so identical values).
template <int XDT, bool REG>
__global__ __launch_bounds__(512) void dqsq_kernel(const void* __restrict__ x, int64_t H,
                                                   const float* __restrict__ ws, const float* __restrict__ as,
                                                   const float* __restrict__ qs, int act_left,
                                                   int8_t* __restrict__ y, float* __restrict__ scale)
{
    __shared__ float red[16];
    const int64_t r = blockIdx.x;
    const int64_t base = r * 2 * H;
    float out[REG ? kDqsqMaxPerThread : 1];
    float amax = 0.0f;
    const float asr = (XDT == CB_DT_INT32) ? as[r] : 1.0f;
    if constexpr (REG) {
#pragma unroll
        for (int u = 0; u < kDqsqMaxPerThread; ++u) {
            const int64_t j = (int64_t)u * blockDim.x + threadIdx.x;
            out[u] = 0.0f;
            if (j < H) {
                out[u] = dqsq_elem<XDT>(x, base, H, j, ws, asr, qs, act_left);
                amax = fmaxf(amax, fabsf(out[u]));
            }
        }
    } else {
        for (int64_t j = threadIdx.x; j < H; j += blockDim.x)
            amax = fmaxf(amax, fabsf(dqsq_elem<XDT>(x, base, H, j, ws, asr, qs, act_left)));
    }
    amax = wave_max(amax);
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = amax;
    __syncthreads();
    amax = 0.0f;
    for (int w = 0; w < nw; ++w) amax = fmaxf(amax, red[w]);
    const float s = fmaxf(amax * kInv127, 1e-12f);
    if (threadIdx.x == 0) scale[r] = s;
    if constexpr (REG) {
#pragma unroll
        for (int u = 0; u < kDqsqMaxPerThread; ++u) {
            const int64_t j = (int64_t)u * blockDim.x + threadIdx.x;
            if (j < H) y[r * H + j] = (int8_t)rint16(fminf(fmaxf(out[u] / s, -128.0f), 127.0f));
        }
    } else {
        for (int64_t j = threadIdx.x; j < H; j += blockDim.x) {
            const float o = dqsq_elem<XDT>(x, base, H, j, ws, asr, qs, act_left);
            y[r * H + j] = (int8_t)rint16(fminf(fmaxf(o / s, -128.0f), 127.0f));
        }
    }
}

// ============================================================================================
// MoeGatingTopKSoftmax
//   Reference semantics (operators/moegatingtopksoftmax/csrc/ops/moe_gating_top_k_softmax/op_kernel/
//   moe_gating_kernel.cpp:15-21): p = softmax(x) in fp32; y = top-k values of p (row dtype);
//   expert_idx = their columns (int32); row_idx[r, j] = j * rows + r; finished[r] -> expert_idx = E.
//   Ties resolve to the lower column (stable order).
// ============================================================================================
template <int DT, int EPL>
__global__ __launch_bounds__(256) void mgt_kernel(const void* __restrict__ x, int64_t rows, int E,
                                                  const uint8_t* __restrict__ finished, int k,
                                                  void* __restrict__ y, int32_t* __restrict__ eidx,
                                                  int32_t* __restrict__ ridx)
{
    const int lane = threadIdx.x & 63;
    const int64_t r = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (r >= rows) return;
    float v[EPL];
    float m = -INFINITY;
#pragma unroll
    for (int u = 0; u < EPL; ++u) {
        const int c = u * 64 + lane;
        v[u] = c < E ? ld_any<DT>(x, r * E + c) : -INFINITY;
        m = fmaxf(m, v[u]);
    }
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < EPL; ++u) {
        const int c = u * 64 + lane;
        v[u] = c < E ? expf(v[u] - m) : -1.0f;  // exp(x - max) >= 0; padding sorts last
        s += c < E ? v[u] : 0.0f;
    }
    s = wave_sum(s);
    const bool fin = finished && finished[r];
    for (int j = 0; j < k; ++j) {
        // wave argmax with the lower column winning ties
        float bv = -2.0f;
        int bc = 0x7fffffff;
#pragma unroll
        for (int u = 0; u < EPL; ++u) {
            const int c = u * 64 + lane;
            if (v[u] > bv || (v[u] == bv && c < bc)) {
                bv = v[u];
                bc = c;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oc = __shfl_xor(bc, o, 64);
            if (ov > bv || (ov == bv && oc < bc)) {
                bv = ov;
                bc = oc;
            }
        }
#pragma unroll
        for (int u = 0; u < EPL; ++u)
            if (u * 64 + lane == bc) v[u] = -2.0f;  // remove the winner
        if (lane == 0) {
            st_any<DT>(y, r * k + j, bv / s);
            eidx[r * k + j] = fin ? E : bc;
            ridx[r * k + j] = (int32_t)((int64_t)j * rows + r);
        }
    }
}

}  // namespace cb

using namespace cb;

// ---------------------------------------------------------------------------------------------
extern "C" int64_t cb_moe_re_routing_workspace_size(int64_t n_ranks, int64_t n_experts)
{
    if (n_ranks <= 0 || n_experts <= 0) return 0;
    return reroute_ws(n_ranks, n_experts).total;
}

extern "C" int cb_moe_re_routing(const void* tokens, int tokens_dtype, int64_t A, int64_t H, const void* counts,
                                 int counts_dtype, int64_t n_ranks, int64_t n_experts, const float* per_token_scales,
                                 void* permute_tokens, float* permute_scales, int32_t* permute_idx,
                                 void* expert_token_num, void* workspace, int64_t workspace_bytes, void* stream)
{
    if (A < 0 || H < 0 || n_ranks < 0 || n_experts < 0) return CB_ERR_SHAPE;
    if (A == 0 || H == 0 || n_ranks == 0 || n_experts == 0) return CB_OK;  // moe_re_routing_plugin.cpp:103-105
    if (tokens_dtype != CB_DT_FLOAT16 && tokens_dtype != CB_DT_BFLOAT16 && tokens_dtype != CB_DT_INT8)
        return CB_ERR_DTYPE;
    if (counts_dtype != CB_DT_INT32 && counts_dtype != CB_DT_INT64) return CB_ERR_DTYPE;
    if (!tokens || !counts || !permute_tokens || !permute_scales || !permute_idx || !expert_token_num)
        return CB_ERR_NULL_POINTER;
    if (A > 0x7fffffffLL || n_ranks > 1024 || n_ranks * n_experts > (1LL << 26)) return CB_ERR_SHAPE;
    const RerouteWs w = reroute_ws(n_ranks, n_experts);
    if (!workspace || workspace_bytes < w.total) return CB_ERR_WORKSPACE;
    hipStream_t st = (hipStream_t)stream;
    uint8_t* wsb = (uint8_t*)workspace;
    int32_t* src = (int32_t*)(wsb + w.src_off);
    int32_t* dst = (int32_t*)(wsb + w.dst_off);
    int32_t* col = (int32_t*)(wsb + w.col_off);
    if (counts_dtype == CB_DT_INT32)
        hipLaunchKernelGGL(mrr_prefix_kernel<int32_t>, dim3(1), dim3(1024), 0, st, (const int32_t*)counts,
                           (int)n_ranks, (int)n_experts, src, dst, col, (int32_t*)expert_token_num);
    else
        hipLaunchKernelGGL(mrr_prefix_kernel<int64_t>, dim3(1), dim3(1024), 0, st, (const int64_t*)counts,
                           (int)n_ranks, (int)n_experts, src, dst, col, (int64_t*)expert_token_num);
    const int64_t esz = tokens_dtype == CB_DT_INT8 ? 1 : 2;
    const int64_t row_bytes = H * esz;
    const int vec = (row_bytes % 16 == 0) && aligned(tokens, 16) && aligned(permute_tokens, 16);
    const int64_t blocks = (A + 3) / 4;
    hipLaunchKernelGGL(mrr_gather_kernel, dim3((unsigned)blocks), dim3(256), 0, st, (const uint8_t*)tokens, A,
                       row_bytes, per_token_scales, src, dst, col, (int)n_ranks, (int)n_experts,
                       (uint8_t*)permute_tokens, permute_scales, permute_idx, vec);
    return check_launch();
}

extern "C" int cb_moe_finalize_routing(const void* expanded_permuted_rows, int dtype, int64_t num_dst, int64_t H,
                                       const int32_t* expanded_src_to_dst_row, int64_t num_rows, int64_t K,
                                       const void* skip1, const void* skip2, const void* bias, int64_t n_bias_rows,
                                       const void* scales, int scales_dtype, const int32_t* expert_for_source_row,
                                       int drop_pad_mode, void* out, void* stream)
{
    if (num_rows < 0 || H < 0 || K <= 0 || num_dst < 0 || n_bias_rows < 0) return CB_ERR_SHAPE;
    if (dtype != CB_DT_FLOAT16 && dtype != CB_DT_BFLOAT16 && dtype != CB_DT_FLOAT32) return CB_ERR_DTYPE;
    if (scales && scales_dtype != CB_DT_FLOAT16 && scales_dtype != CB_DT_BFLOAT16 && scales_dtype != CB_DT_FLOAT32)
        return CB_ERR_DTYPE;
    if (num_rows == 0 || H == 0) return CB_OK;
    if (!expanded_permuted_rows || !expanded_src_to_dst_row || !out) return CB_ERR_NULL_POINTER;
    if (bias && !expert_for_source_row) bias = nullptr;  // the bias is applied only with the expert table
    if (num_rows > 0x7fffffffLL) return CB_ERR_SHAPE;
    MfrArgs a;
    std::memset(&a, 0, sizeof(a));
    a.epr = expanded_permuted_rows;
    a.esdr = expanded_src_to_dst_row;
    a.skip1 = skip1;
    a.skip2 = skip2;
    a.bias = bias;
    a.scales = scales;
    a.expert = expert_for_source_row;
    a.out = out;
    a.num_dst = num_dst;
    a.num_rows = num_rows;
    a.H = H;
    a.K = K;
    a.E = bias ? n_bias_rows : 0;
    const int mode = drop_pad_mode < 0 ? 0 : (drop_pad_mode > 3 ? 3 : drop_pad_mode);
    a.col_mode = mode <= 1;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)num_rows), block(256);
    const int sdt = scales ? scales_dtype : dtype;
#define CB_MFR(DTV, SDTV) hipLaunchKernelGGL((mfr_kernel<DTV, SDTV>), grid, block, 0, st, a)
#define CB_MFR_S(DTV)                                                                              \
    do {                                                                                           \
        if (sdt == CB_DT_FLOAT32) CB_MFR(DTV, CB_DT_FLOAT32);                                      \
        else if (sdt == CB_DT_BFLOAT16) CB_MFR(DTV, CB_DT_BFLOAT16);                               \
        else CB_MFR(DTV, CB_DT_FLOAT16);                                                           \
    } while (0)
    if (dtype == CB_DT_FLOAT32) CB_MFR_S(CB_DT_FLOAT32);
    else if (dtype == CB_DT_BFLOAT16) CB_MFR_S(CB_DT_BFLOAT16);
    else CB_MFR_S(CB_DT_FLOAT16);
#undef CB_MFR_S
#undef CB_MFR
    return check_launch();
}

extern "C" int cb_dequant_swiglu_quant(const void* x, int x_dtype, int64_t M, int64_t N2, const float* weight_scale,
                                       const float* activation_scale, const float* quant_scale, int activate_left,
                                       int8_t* y, float* scale, void* stream)
{
    if (M < 0 || N2 < 0) return CB_ERR_SHAPE;
    if (N2 % 2 != 0) return CB_ERR_N_ODD;
    if (M == 0 || N2 == 0) return CB_OK;
    if (x_dtype != CB_DT_INT32 && x_dtype != CB_DT_FLOAT16 && x_dtype != CB_DT_BFLOAT16) return CB_ERR_DTYPE;
    if (x_dtype == CB_DT_INT32 && (!weight_scale || !activation_scale)) return CB_ERR_NULL_POINTER;
    if (x_dtype != CB_DT_INT32 && (weight_scale || activation_scale)) return CB_ERR_SCALE_LEN;
    if (!x || !y || !scale) return CB_ERR_NULL_POINTER;
    const int64_t H = N2 / 2;
    if (M > 0x7fffffffLL) return CB_ERR_SHAPE;
    const bool reg = H <= (int64_t)kDqsqMaxPerThread * 512;
    int threads = (int)((H + kDqsqMaxPerThread - 1) / kDqsqMaxPerThread);
    threads = (threads + 63) / 64 * 64;
    threads = threads < 64 ? 64 : (threads > 512 ? 512 : threads);
    if (!reg) threads = 512;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)M), block(threads);
#define CB_DQSQ(XDTV)                                                                              \
    do {                                                                                           \
        if (reg)                                                                                   \
            hipLaunchKernelGGL((dqsq_kernel<XDTV, true>), grid, block, 0, st, x, H, weight_scale,   \
                               activation_scale, quant_scale, activate_left, y, scale);            \
        else                                                                                       \
            hipLaunchKernelGGL((dqsq_kernel<XDTV, false>), grid, block, 0, st, x, H, weight_scale,  \
                               activation_scale, quant_scale, activate_left, y, scale);            \
    } while (0)
    if (x_dtype == CB_DT_INT32) CB_DQSQ(CB_DT_INT32);
    else if (x_dtype == CB_DT_BFLOAT16) CB_DQSQ(CB_DT_BFLOAT16);
    else CB_DQSQ(CB_DT_FLOAT16);
#undef CB_DQSQ
    return check_launch();
}

extern "C" int cb_moe_gating_top_k_softmax(const void* x, int dtype, int64_t rows, int64_t E,
                                           const uint8_t* finished, int64_t k, void* y, int32_t* expert_idx,
                                           int32_t* row_idx, void* stream)
{
    if (dtype != CB_DT_FLOAT32 && dtype != CB_DT_FLOAT16 && dtype != CB_DT_BFLOAT16) return CB_ERR_DTYPE;
    if (E <= 0) return CB_ERR_EMPTY;
    if (k <= 0 || k > E) return CB_ERR_SHAPE;
    if (rows <= 0) return CB_ERR_EMPTY;
    if (E > 2048 || rows > 0x7fffffffLL) return CB_ERR_SHAPE;
    if (!x || !y || !expert_idx || !row_idx) return CB_ERR_NULL_POINTER;
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    const int epl = (int)((E + 63) / 64);
#define CB_MGT(DTV, EPLV)                                                                          \
    hipLaunchKernelGGL((mgt_kernel<DTV, EPLV>), grid, block, 0, st, x, rows, (int)E, finished, (int)k, y,   \
                       expert_idx, row_idx)
#define CB_MGT_E(DTV)                                                                              \
    do {                                                                                           \
        if (epl <= 1) CB_MGT(DTV, 1);                                                              \
        else if (epl <= 2) CB_MGT(DTV, 2);                                                         \
        else if (epl <= 4) CB_MGT(DTV, 4);                                                         \
        else if (epl <= 8) CB_MGT(DTV, 8);                                                         \
        else if (epl <= 16) CB_MGT(DTV, 16);                                                       \
        else CB_MGT(DTV, 32);                                                                      \
    } while (0)
    if (dtype == CB_DT_FLOAT32) CB_MGT_E(CB_DT_FLOAT32);
    else if (dtype == CB_DT_BFLOAT16) CB_MGT_E(CB_DT_BFLOAT16);
    else CB_MGT_E(CB_DT_FLOAT16);
#undef CB_MGT_E
#undef CB_MGT
    return check_launch();
}
