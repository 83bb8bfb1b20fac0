// moe_routing.hip - the operators on either side of the MoE-FFN path, for gfx950:
//   cb_moe_re_routing            token permutation rank-major -> expert-major (feeds GMSQ)
//   cb_moe_finalize_routing      weighted combine of expert outputs + skips + bias (after the
//                                down-projection)
//   cb_dequant_swiglu_quant      standalone dequant + SwiGLU + per-token int8 quant
//   cb_moe_gating_top_k_softmax  softmax + top-k routing producer
// All four are HBM-bound gather / row kernels: rows are moved with 16-byte accesses, per-row
// reductions are wave / workgroup shuffles, and nothing is staged through host memory.
#include <cstring>
#include <type_traits>

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

// LDS version of the prefix pass for count matrices of at most kMrrLdsCells cells (n, e <= 1024):
// row and column running sums in LDS, then two Hillis-Steele scans over the row and column totals.
constexpr int kMrrLdsCells = 8192;

// Exclusive scan of buf[0, n) (n <= 1024) by the whole block: Hillis-Steele steps ping-ponging
// between buf and tmp, then a shift by one.  Every thread of the block must call it.
__device__ __forceinline__ void block_excl_scan(int32_t* buf, int n, int32_t* tmp)
{
    int32_t* a = buf;
    int32_t* b = tmp;
    for (int off = 1; off < n; off <<= 1) {
        for (int t = threadIdx.x; t < n; t += blockDim.x) b[t] = a[t] + (t >= off ? a[t - off] : 0);
        __syncthreads();
        int32_t* c = a;
        a = b;
        b = c;
    }
    if (a == buf) {  // the shift below must read from a buffer other than buf
        for (int t = threadIdx.x; t < n; t += blockDim.x) tmp[t] = buf[t];
        __syncthreads();
        a = tmp;
    }
    for (int t = threadIdx.x; t < n; t += blockDim.x) buf[t] = t ? a[t - 1] : 0;
    __syncthreads();
}

template <typename CT>
__global__ __launch_bounds__(1024) void mrr_prefix_lds_kernel(const CT* __restrict__ cnt, int n, int e,
                                                              int32_t* __restrict__ src_start,
                                                              int32_t* __restrict__ dst_start,
                                                              int32_t* __restrict__ col_start, CT* __restrict__ etn)
{
    __shared__ int32_t c[kMrrLdsCells];
    __shared__ int32_t rs[1024], cs[1024], rtot[1024], ctot[1024], tmp[1025];
    const int cells = n * e;
    for (int t = threadIdx.x; t < cells; t += blockDim.x) c[t] = (int32_t)cnt[t];
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int32_t run = 0;
        for (int j = 0; j < e; ++j) run += c[i * e + j];
        rtot[i] = run;
        rs[i] = run;
    }
    for (int j = threadIdx.x; j < e; j += blockDim.x) {
        int32_t run = 0;
        for (int i = 0; i < n; ++i) run += c[i * e + j];
        ctot[j] = run;
        cs[j] = run;
    }
    __syncthreads();
    block_excl_scan(rs, n, tmp);  // rs[i] = row start
    block_excl_scan(cs, e, tmp);  // cs[j] = column start
    for (int j = threadIdx.x; j < e; j += blockDim.x) {
        etn[j] = (CT)ctot[j];
        col_start[j] = cs[j];
    }
    if (threadIdx.x == 0) col_start[e] = e ? cs[e - 1] + ctot[e - 1] : 0;
    // per-row exclusive prefix along experts, per-column exclusive prefix along ranks
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        int32_t run = rs[i];
        for (int j = 0; j < e; ++j) {
            src_start[i * e + j] = run;
            run += c[i * e + j];
        }
    }
    for (int j = threadIdx.x; j < e; j += blockDim.x) {
        int32_t run = cs[j];
        for (int i = 0; i < n; ++i) {
            dst_start[i * e + j] = run;
            run += c[i * e + j];
        }
    }
}

// One thread per destination row: locate its (rank, expert) cell by two binary searches over the
// prefix tables and record the source row (permute_idx) and its scale.
__global__ __launch_bounds__(256) void mrr_route_kernel(int64_t a, const float* __restrict__ scales,
                                                        const int32_t* __restrict__ src_start,
                                                        const int32_t* __restrict__ dst_start,
                                                        const int32_t* __restrict__ col_start, int n, int e,
                                                        float* __restrict__ out_sc, int32_t* __restrict__ out_idx)
{
    const int64_t d = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
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
    const bool ok = src >= 0 && src < a;
    out_idx[d] = ok ? (int32_t)src : -1;  // -1 only for inconsistent counts (sum > A): row not copied
    out_sc[d] = (ok && scales) ? scales[src] : 0.0f;
}

// One wave per destination row: copy tokens[permute_idx[d]] into row d.
__global__ __launch_bounds__(256) void mrr_copy_kernel(const uint8_t* __restrict__ tokens, int64_t a,
                                                       int64_t row_bytes, const int32_t* __restrict__ col_start,
                                                       int e, uint8_t* __restrict__ out_tok,
                                                       int32_t* __restrict__ out_idx, int vec16)
{
    const int lane = threadIdx.x & 63;
    const int64_t d = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int64_t total = col_start[e];
    if (d >= a || d >= total) return;
    const int64_t src = out_idx[d];
    if (src < 0) return;
    const uint8_t* s = tokens + src * row_bytes;
    uint8_t* o = out_tok + d * row_bytes;
    if (vec16) {
        // batches of 8 independent 16-byte loads per lane before their stores; offsets past the
        // row read zeros and drop the store, so no lane branches around the loads
        const int64_t nv = row_bytes >> 4;
        const auto rs = row_rsrc(s, (uint32_t)row_bytes);
        const auto ro = row_rsrc(o, (uint32_t)row_bytes);
        for (int64_t v0 = 0; v0 < nv; v0 += 8 * 64) {
            iv4 t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = row_load(rs, (uint32_t)(v0 + u * 64 + lane) * 16u);
#pragma unroll
            for (int u = 0; u < 8; ++u) row_store(t[u], ro, (uint32_t)(v0 + u * 64 + lane) * 16u);
        }
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

// 16-byte vectors of V elements (V = 4 fp32 / int32, 8 fp16 / bf16) unpacked to fp32.
template <int DT>
struct Vec16 {
    static constexpr int V = (DT == CB_DT_FLOAT32 || DT == CB_DT_INT32) ? 4 : 8;
    __device__ static __forceinline__ void unpack(const iv4 r, float* f)
    {
        if constexpr (DT == CB_DT_FLOAT32) {
#pragma unroll
            for (int q = 0; q < 4; ++q) f[q] = __int_as_float(r[q]);
        } else if constexpr (DT == CB_DT_INT32) {
#pragma unroll
            for (int q = 0; q < 4; ++q) f[q] = (float)r[q];
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32 w = (u32)r[q];
                f[2 * q] = DT == CB_DT_BFLOAT16 ? bf16_to_f32((uint16_t)(w & 0xffffu)) : f16_to_f32((uint16_t)(w & 0xffffu));
                f[2 * q + 1] = DT == CB_DT_BFLOAT16 ? bf16_to_f32((uint16_t)(w >> 16)) : f16_to_f32((uint16_t)(w >> 16));
            }
        }
    }
    __device__ static __forceinline__ iv4 pack(const float* f)
    {
        iv4 r;
        if constexpr (DT == CB_DT_FLOAT32) {
#pragma unroll
            for (int q = 0; q < 4; ++q) r[q] = __float_as_int(f[q]);
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const u32 lo = DT == CB_DT_BFLOAT16 ? f32_to_bf16(f[2 * q]) : f32_to_f16(f[2 * q]);
                const u32 hi = DT == CB_DT_BFLOAT16 ? f32_to_bf16(f[2 * q + 1]) : f32_to_f16(f[2 * q + 1]);
                r[q] = (int)(lo | (hi << 16));
            }
        }
        return r;
    }
};

// Vectorised MoeFinalizeRouting: each thread owns 16-byte column vectors of one output row.  The
// row's K slot descriptors (source row or -1, bias row or -1, scale) are staged once in LDS; every
// load then goes through a per-slot buffer resource whose size is 0 for an absent slot, so the
// skip rows and 8 expert rows (and their bias rows) are issued back to back without branches.
// The terms are added in ascending k, skipping dropped slots: the scalar kernel's order.
constexpr int kMfrMaxK = 64;

template <int DT, int SDT>
__global__ __launch_bounds__(512) void mfr_vec_kernel(const MfrArgs a)
{
    using VT = Vec16<DT>;
    constexpr int V = VT::V;
    __shared__ int64_t s_p[kMfrMaxK + 8];
    __shared__ int32_t s_e[kMfrMaxK + 8];
    __shared__ float s_sc[kMfrMaxK + 8];
    const int64_t i = blockIdx.x;
    const int64_t H = a.H, K = a.K;
    const int64_t nv = H / V;
    const uint32_t rb = (uint32_t)(H * (DT == CB_DT_FLOAT32 ? 4 : 2));
    const int64_t kpad = (K + 7) / 8 * 8;
    for (int t = threadIdx.x; t < kpad; t += blockDim.x) {
        int64_t p = -1;
        int32_t e = -1;
        float sc = 1.0f;
        if (t < K) {
            const int64_t q = a.esdr[a.col_mode ? (int64_t)t * a.num_rows + i : i * K + t];
            p = (q >= 0 && q < a.num_dst) ? q : -1;
            if (a.bias) {
                const int64_t eid = a.expert[i * K + t];
                e = (eid >= 0 && eid < a.E) ? (int32_t)eid : -1;
            }
            if (a.scales) sc = ld_any<SDT>(a.scales, i * K + t);
        }
        s_p[t] = p;
        s_e[t] = e;
        s_sc[t] = sc;
    }
    __syncthreads();
    const char* epr = (const char*)a.epr;
    const auto r_sk1 = row_rsrc(a.skip1 ? (const char*)a.skip1 + i * rb : epr, a.skip1 ? rb : 0);
    const auto r_sk2 = row_rsrc(a.skip2 ? (const char*)a.skip2 + i * rb : epr, a.skip2 ? rb : 0);
    const bool has_bias = a.bias != nullptr, has_scales = a.scales != nullptr;
    for (int64_t cv = threadIdx.x; cv < nv; cv += blockDim.x) {
        const uint32_t off = (uint32_t)cv * 16u;
        const iv4 sk1 = row_load(r_sk1, off);
        const iv4 sk2 = row_load(r_sk2, off);
        float acc[V];
        for (int64_t k0 = 0; k0 < K; k0 += 8) {
            iv4 raw[8], braw[8];
            int64_t pk[8];
            int32_t ek[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                pk[u] = uniform64(s_p[k0 + u]);
                ek[u] = (int32_t)__builtin_amdgcn_readfirstlane((uint32_t)s_e[k0 + u]);
                raw[u] = row_load(row_rsrc(pk[u] >= 0 ? epr + pk[u] * rb : epr, pk[u] >= 0 ? rb : 0), off);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const char* bb = (const char*)a.bias;
                braw[u] = row_load(row_rsrc(ek[u] >= 0 ? bb + (int64_t)ek[u] * rb : epr, ek[u] >= 0 ? rb : 0), off);
            }
            if (k0 == 0) {  // the skips, consumed once the first expert rows are in flight
                VT::unpack(sk1, acc);  // zeros when skip1 is absent
                if (a.skip2) {
                    float t2[V];
                    VT::unpack(sk2, t2);
#pragma unroll
                    for (int q = 0; q < V; ++q) acc[q] = acc[q] + t2[q];
                }
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                if (pk[u] < 0) continue;  // dropped slot (or past K): no term
                float t[V];
                VT::unpack(raw[u], t);
                if (has_bias && ek[u] >= 0) {
                    float b[V];
                    VT::unpack(braw[u], b);
#pragma unroll
                    for (int q = 0; q < V; ++q) t[q] = t[q] + b[q];
                }
                if (has_scales) {
                    const float sc = s_sc[k0 + u];
#pragma unroll
                    for (int q = 0; q < V; ++q) t[q] = t[q] * sc;
                }
#pragma unroll
                for (int q = 0; q < V; ++q) acc[q] = acc[q] + t[q];
            }
        }
        __builtin_nontemporal_store(VT::pack(acc), (iv4*)a.out + i * nv + cv);
    }
}

// Threads per block for n work items of one row: a multiple of 64 in [64, 512] that wastes the
// fewest lanes over the row's passes, preferring more threads on ties.
static int row_threads(int64_t n, int64_t max_passes = 1LL << 40)
{
    int best = 512;
    int64_t best_waste = -1;
    for (int t = 512; t >= 64; t -= 64) {
        const int64_t passes = (n + t - 1) / t;
        if (passes > max_passes) continue;
        const int64_t waste = passes * t - n;
        if (best_waste < 0 || waste < best_waste) {
            best = t;
            best_waste = waste;
        }
    }
    return best;
}

// ============================================================================================
// DequantSwigluQuant
//   Reference semantics (operators/dequantswigluquant/csrc/ops/dequant_swiglu_quant/op_kernel/
//   dqsq_kernel.cpp:15-27 and the operation order of :336-427, 476-524):
//     A = f32(x[:, :H]) [* weight_scale[:H]], B = f32(x[:, H:]) [* weight_scale[H:]]   (int32 x)
//     the non-gate half *= quant_scale                     (when given)
//     A *= activation_scale[row], B *= activation_scale[row] (int32 x)
//     out = (A * B) / (1 + exp(-G)),  G = B (activate_left false) or A (true)
//     s = max(max_j |out| * (1/127), 1e-12);  y = rint16(clamp(out * (1/s), -128, 127))
//   The quotient by s is taken as a product with the row's reciprocal, the reference's form for
//   long rows (dqsq_kernel.cpp:489-505); exp and the SiLU reciprocal use the hardware v_exp_f32 /
//   v_rcp_f32 (about 1 ulp), so an int8 output can differ from a correctly rounded evaluation by
//   one step where the scaled value lies within an ulp of a rounding boundary.
// ============================================================================================
template <int XDT>
__device__ __forceinline__ float ld_x(const void* x, int64_t i)
{
    if constexpr (XDT == CB_DT_INT32) return (float)((const int32_t*)x)[i];
    else if constexpr (XDT == CB_DT_BFLOAT16) return bf16_to_f32(((const uint16_t*)x)[i]);
    else return f16_to_f32(((const uint16_t*)x)[i]);
}

constexpr int kDqsqMaxPerThread = 16;
// values per thread of the vectorised DequantSwigluQuant row (sets its threads per row)
constexpr int kDqsqEpt = 4;

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
    return (A * B) * __builtin_amdgcn_rcpf(1.0f + __expf(-G));
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
    const float inv = 1.0f / s;
    if (threadIdx.x == 0) scale[r] = s;
    if constexpr (REG) {
#pragma unroll
        for (int u = 0; u < kDqsqMaxPerThread; ++u) {
            const int64_t j = (int64_t)u * blockDim.x + threadIdx.x;
            if (j < H) y[r * H + j] = (int8_t)rint16_inrange(fminf(fmaxf(out[u] * inv, -128.0f), 127.0f));
        }
    } else {
        for (int64_t j = threadIdx.x; j < H; j += blockDim.x) {
            const float o = dqsq_elem<XDT>(x, base, H, j, ws, asr, qs, act_left);
            y[r * H + j] = (int8_t)rint16_inrange(fminf(fmaxf(o * inv, -128.0f), 127.0f));
        }
    }
}

// Vectorised DequantSwigluQuant: a persistent grid walks the rows (row = blockIdx.x + i * gridDim.x),
// so the weight_scale / quant_scale slices of a thread stay in registers across rows; both halves
// arrive as 16-byte buffer loads (lanes past the row read zeros, which give out = 0 and leave the
// row max unchanged) and the next row's loads are issued before the current row is reduced.
// QS / LEFT fix the optional quant_scale and activate_left at compile time.  Per element the
// arithmetic is dqsq_elem's.
template <int XDT, int NV, bool QS, bool LEFT>
__global__ __launch_bounds__(512) void dqsq_vec_kernel(const void* __restrict__ x, int64_t M, int64_t H,
                                                       const float* __restrict__ ws, const float* __restrict__ as,
                                                       const float* __restrict__ qs, int8_t* __restrict__ y,
                                                       float* __restrict__ scale)
{
    using VT = Vec16<XDT>;
    constexpr int V = VT::V;
    constexpr bool I32 = XDT == CB_DT_INT32;
    constexpr int ESZ = (XDT == CB_DT_INT32) ? 4 : 2;
    __shared__ float red[2][16];
    const int64_t nvh = H / V;
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const uint32_t hb = (uint32_t)(H * ESZ);  // bytes of one half row
    // per-thread column constants (zeros for lanes past the row)
    float wa[I32 ? NV : 1][I32 ? V : 1], wb[I32 ? NV : 1][I32 ? V : 1], qv[QS ? NV : 1][QS ? V : 1];
    uint32_t offa[NV], offy[NV];
    const auto r_ws = row_rsrc(ws ? (const void*)ws : x, I32 ? (uint32_t)(2 * H * 4) : 0u);
    const auto r_qs = row_rsrc(qs ? (const void*)qs : x, QS ? (uint32_t)(H * 4) : 0u);
#pragma unroll
    for (int u = 0; u < NV; ++u) {
        const int64_t cv = (int64_t)u * blockDim.x + threadIdx.x;
        const bool ok = cv < nvh;
        offa[u] = ok ? (uint32_t)cv * 16u : kOffNone;
        offy[u] = ok ? (uint32_t)(cv * V) : kOffNone;
        if constexpr (I32) {
            const uint32_t wo = ok ? (uint32_t)(cv * V * 4) : kOffNone;
            const iv4 w0 = row_load(r_ws, wo), w1 = row_load(r_ws, ok ? wo + (uint32_t)(H * 4) : kOffNone);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                wa[u][q] = __int_as_float(w0[q]);
                wb[u][q] = __int_as_float(w1[q]);
            }
        }
        if constexpr (QS) {
#pragma unroll
            for (int q4 = 0; q4 < V / 4; ++q4) {
                const iv4 qq = row_load(r_qs, ok ? (uint32_t)((cv * V + q4 * 4) * 4) : kOffNone);
#pragma unroll
                for (int q = 0; q < 4; ++q) qv[u][q4 * 4 + q] = __int_as_float(qq[q]);
            }
        }
    }
    iv4 ra[NV], rb[NV];
    auto load_row = [&](int64_t r) {
        const auto rx = row_rsrc((const char*)x + r * 2 * (int64_t)hb, 2 * hb);
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            ra[u] = row_load(rx, offa[u]);
            rb[u] = row_load(rx, offa[u] == kOffNone ? kOffNone : offa[u] + hb);
        }
    };
    int64_t r = blockIdx.x;
    if (r < M) load_row(r);
    for (int parity = 0; r < M; r += gridDim.x, parity ^= 1) {
        float out[NV][V];
        float amax = 0.0f;
        const float asr = I32 ? as[r] : 1.0f;
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            float A[V], B[V];
            VT::unpack(ra[u], A);
            VT::unpack(rb[u], B);
#pragma unroll
            for (int q = 0; q < V; ++q) {
                if constexpr (I32) {
                    A[q] = A[q] * wa[u][q];
                    B[q] = B[q] * wb[u][q];
                }
                if constexpr (QS) {
                    if constexpr (LEFT) B[q] = B[q] * qv[u][q];
                    else A[q] = A[q] * qv[u][q];
                }
                if constexpr (I32) {
                    A[q] = A[q] * asr;
                    B[q] = B[q] * asr;
                }
                const float G = LEFT ? A[q] : B[q];
                out[u][q] = (A[q] * B[q]) * __builtin_amdgcn_rcpf(1.0f + __expf(-G));
                amax = fmaxf(amax, fabsf(out[u][q]));
            }
        }
        const int64_t rn = r + gridDim.x;
        if (rn < M) load_row(rn);  // next row in flight during the reduction and the stores
        amax = wave_max(amax);
        // double-buffered partials: one barrier per row suffices
        if ((threadIdx.x & 63) == 0) red[parity][wave] = amax;
        __syncthreads();
        amax = 0.0f;
        for (int w = 0; w < nw; ++w) amax = fmaxf(amax, red[parity][w]);
        const float s = fmaxf(amax * kInv127, 1e-12f);
        const float inv = 1.0f / s;
        if (threadIdx.x == 0) scale[r] = s;
        const auto ry = row_rsrc(y + r * H, (uint32_t)H);
#pragma unroll
        for (int u = 0; u < NV; ++u) {
            u32 w[V / 4];
#pragma unroll
            for (int q4 = 0; q4 < V / 4; ++q4) {
                int8_t b[4];
#pragma unroll
                for (int t = 0; t < 4; ++t)
                    b[t] = (int8_t)rint16_inrange(fminf(fmaxf(out[u][q4 * 4 + t] * inv, -128.0f), 127.0f));
                w[q4] = pack4_i8(b[0], b[1], b[2], b[3]);
            }
            if constexpr (V == 4) {
                __builtin_amdgcn_raw_buffer_store_b32(w[0], ry, offy[u], 0, 2);
            } else {
                typedef u32 u2v __attribute__((ext_vector_type(2)));
                u2v pw;
                pw[0] = w[0];
                pw[1] = w[1];
                __builtin_amdgcn_raw_buffer_store_b64(pw, ry, offy[u], 0, 2);
            }
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
// Row reductions over LPR consecutive lanes (LPR = 16 or 64) with DPP moves, no LDS traffic:
// two quad permutations and two row rotations reduce each 16-lane row; for LPR = 64 the four row
// results are then combined through readlane.
template <bool MAX>
__device__ __forceinline__ float dpp_op(float a, float b) { return MAX ? fmaxf(a, b) : a + b; }

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v)
{
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

template <int LPR, bool MAX>
__device__ __forceinline__ float row_reduce(float v)
{
    v = dpp_op<MAX>(v, dpp_mov<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = dpp_op<MAX>(v, dpp_mov<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = dpp_op<MAX>(v, dpp_mov<0x124>(v));  // row_ror 4
    v = dpp_op<MAX>(v, dpp_mov<0x128>(v));  // row_ror 8
    if constexpr (LPR == 64) {
        const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
        const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
        const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
        const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
        v = dpp_op<MAX>(dpp_op<MAX>(r0, r1), dpp_op<MAX>(r2, r3));
    }
    return v;
}

// Row maximum of round candidates: exp(x - max) >= 0 or the -1 sentinel.  Compared as signed
// integers these order as the floats do (non-negative floats by their bits, -1 below them), and
// the DPP moves fuse into v_max_i32 without the float path's canonicalising max.
template <int CTRL>
__device__ __forceinline__ int dpp_imax(int v)
{
    return max(v, __builtin_amdgcn_update_dpp((int)0x80000000, v, CTRL, 0xf, 0xf, false));
}

template <int LPR>
__device__ __forceinline__ float row_max_candidates(float f)
{
    int v = __float_as_int(f);
    v = dpp_imax<0xB1>(v);   // quad_perm [1, 0, 3, 2]
    v = dpp_imax<0x4E>(v);   // quad_perm [2, 3, 0, 1]
    v = dpp_imax<0x124>(v);  // row_ror 4
    v = dpp_imax<0x128>(v);  // row_ror 8
    if constexpr (LPR == 64) {
        const int r0 = __builtin_amdgcn_readlane(v, 0), r1 = __builtin_amdgcn_readlane(v, 16);
        const int r2 = __builtin_amdgcn_readlane(v, 32), r3 = __builtin_amdgcn_readlane(v, 48);
        v = max(max(r0, r1), max(r2, r3));
    }
    return __int_as_float(v);
}

// One row per LPR lanes; lane `sub` of a row owns the EPL consecutive columns [sub*EPL, sub*EPL+EPL).
// Each of the k rounds takes every lane's best remaining value (lowest column on ties), reduces the
// row maximum, and lets the lowest lane holding it (hence the lowest column) emit it: the order of a
// stable descending sort.  Every lane of the wave stays active for the DPP moves.
//
// A lane keeps its next MGT_LIST values in emission order (descending, lower column first on ties),
// built once by insertion (MGT_LIST = k for k <= 2, else 4).  A win pops the head; a lane whose
// list a win empties rebuilds it from the columns after the one it emitted last (a wave-uniform
// branch, rare for MGT_LIST 4: a lane must win 4 of the k rounds), except after the last round.
// For k <= LPR the round's value and column go to row lane j (the column read from the winner
// with ds_bpermute), and after the rounds each of the first k lanes of the row divides once and
// stores its output; larger k store from the winner in each round.
template <int DT, int LPR, int EPL, bool VLD, int MGT_LIST>
__global__ __launch_bounds__(256) void mgt_kernel(const void* __restrict__ x, int64_t rows, int E,
                                                  const uint8_t* __restrict__ finished, int k,
                                                  void* __restrict__ y, int32_t* __restrict__ eidx,
                                                  int32_t* __restrict__ ridx)
{
    constexpr int RPW = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int sub = lane % LPR, grp = lane / LPR;
    const int64_t r = ((int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * RPW + grp;
    const bool live = r < rows;
    const int c0 = sub * EPL;
    float v[EPL];
    if constexpr (VLD) {
        // E == LPR * EPL and 16-byte aligned rows: whole-vector loads
        using VT = Vec16<DT>;
        constexpr int V = VT::V;
        static_assert(EPL % V == 0, "vector load needs whole vectors per lane");
        const iv4* src = (const iv4*)x + ((live ? r : 0) * E + c0) / V;
#pragma unroll
        for (int q = 0; q < EPL / V; ++q) {
            const iv4 w = src[q];
            VT::unpack(w, v + q * V);
        }
        if (!live) {
#pragma unroll
            for (int u = 0; u < EPL; ++u) v[u] = -INFINITY;
        }
    } else {
#pragma unroll
        for (int u = 0; u < EPL; ++u) v[u] = (live && c0 + u < E) ? ld_any<DT>(x, r * E + c0 + u) : -INFINITY;
    }
    float m = v[0];
#pragma unroll
    for (int u = 1; u < EPL; ++u) m = fmaxf(m, v[u]);
    m = row_reduce<LPR, true>(m);
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < EPL; ++u) {
        const bool in = live && c0 + u < E;
        v[u] = in ? __expf(v[u] - m) : -1.0f;  // exp(x - max) >= 0: padding sorts last
        s += in ? v[u] : 0.0f;
    }
    s = row_reduce<LPR, false>(s);
    const bool fin = live && finished && finished[r];
    constexpr int T = EPL < MGT_LIST ? EPL : MGT_LIST;
    float tv[T];
    int tu[T];
    // the lane's best T values among the slots after (lv, lu) in emission order (every slot when
    // `all` is true_type); padding and an empty list entry are -1, below every exp(x - max) >= 0
    auto fill = [&](auto all, const float lv, const int lu) {
#pragma unroll
        for (int t = 0; t < T; ++t) {
            tv[t] = -1.0f;
            tu[t] = 0;
        }
#pragma unroll
        for (int u = 0; u < EPL; ++u) {
            float x = v[u];
            if constexpr (!decltype(all)::value) x = (v[u] < lv || (v[u] == lv && u > lu)) ? x : -1.0f;
            bool g[T];
#pragma unroll
            for (int t = 0; t < T; ++t) g[t] = x > tv[t];  // strict: the lower slot stays first on ties
#pragma unroll
            for (int t = T - 1; t > 0; --t) {
                tv[t] = g[t - 1] ? tv[t - 1] : (g[t] ? x : tv[t]);
                tu[t] = g[t - 1] ? tu[t - 1] : (g[t] ? u : tu[t]);
            }
            tv[0] = g[0] ? x : tv[0];
            tu[0] = g[0] ? u : tu[0];
        }
    };
    fill(std::true_type{}, 0.0f, 0);
    float lv = 0.0f;
    int lu = 0;
    // the row's winner (row lane wsub, the lowest holding the row maximum); the winner pops its
    // head, and a lane whose list that empties refills it (a lane without values left rebuilds an
    // empty list, which is harmless) unless it was the last round
    auto winner = [&](const float mrow) {
        const unsigned long long hit = __ballot(tv[0] == mrow);
        if constexpr (LPR == 64) return __ffsll((long long)hit) - 1;
        else return __ffs((unsigned)(hit >> (grp * LPR)) & ((1u << LPR) - 1u)) - 1;
    };
    auto pop = [&](const bool win, const int j) {
        if (win) {
            lv = tv[0];
            lu = tu[0];
#pragma unroll
            for (int t = 0; t + 1 < T; ++t) {
                tv[t] = tv[t + 1];
                tu[t] = tu[t + 1];
            }
            tv[T - 1] = -1.0f;
        }
        const bool refill = win && tv[0] < 0.0f;
        if (j + 1 < k && __ballot(refill) != 0ull) {
            if (refill) fill(std::false_type{}, lv, lu);
        }
    };
    if (k <= LPR) {
        float ov = 0.0f;
        int oc = 0;
        for (int j = 0; j < k; ++j) {
            const float mrow = row_max_candidates<LPR>(tv[0]);
            const int wsub = winner(mrow);
            const int col = __builtin_amdgcn_ds_bpermute((grp * LPR + wsub) << 2, c0 + tu[0]);
            ov = sub == j ? mrow : ov;
            oc = sub == j ? col : oc;
            pop(sub == wsub, j);
        }
        if (live && sub < k) {
            st_any<DT>(y, r * k + sub, ov / s);
            eidx[r * k + sub] = fin ? E : oc;
            ridx[r * k + sub] = (int32_t)((int64_t)sub * rows + r);
        }
    } else {
        for (int j = 0; j < k; ++j) {
            const float mrow = row_max_candidates<LPR>(tv[0]);
            const bool win = sub == winner(mrow);
            if (win && live) {
                st_any<DT>(y, r * k + j, tv[0] / s);
                eidx[r * k + j] = fin ? E : c0 + tu[0];
                ridx[r * k + j] = (int32_t)((int64_t)j * rows + r);
            }
            pop(win, j);
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
    if (!grid_fits((A + 3) / 4, 256)) return CB_ERR_SHAPE;  // the copy kernel: 4 rows per block
    TimedLaunch timed(st);
    uint8_t* wsb = (uint8_t*)workspace;
    int32_t* src = (int32_t*)(wsb + w.src_off);
    int32_t* dst = (int32_t*)(wsb + w.dst_off);
    int32_t* col = (int32_t*)(wsb + w.col_off);
    const bool lds = n_ranks <= 1024 && n_experts <= 1024 && n_ranks * n_experts <= kMrrLdsCells;
    if (lds && counts_dtype == CB_DT_INT32)
        hipLaunchKernelGGL(mrr_prefix_lds_kernel<int32_t>, dim3(1), dim3(1024), 0, st, (const int32_t*)counts,
                           (int)n_ranks, (int)n_experts, src, dst, col, (int32_t*)expert_token_num);
    else if (lds)
        hipLaunchKernelGGL(mrr_prefix_lds_kernel<int64_t>, dim3(1), dim3(1024), 0, st, (const int64_t*)counts,
                           (int)n_ranks, (int)n_experts, src, dst, col, (int64_t*)expert_token_num);
    else if (counts_dtype == CB_DT_INT32)
        hipLaunchKernelGGL(mrr_prefix_kernel<int32_t>, dim3(1), dim3(1024), 0, st, (const int32_t*)counts,
                           (int)n_ranks, (int)n_experts, src, dst, col, (int32_t*)expert_token_num);
    else
        hipLaunchKernelGGL(mrr_prefix_kernel<int64_t>, dim3(1), dim3(1024), 0, st, (const int64_t*)counts,
                           (int)n_ranks, (int)n_experts, src, dst, col, (int64_t*)expert_token_num);
    const int64_t esz = tokens_dtype == CB_DT_INT8 ? 1 : 2;
    const int64_t row_bytes = H * esz;
    const int vec = (row_bytes % 16 == 0) && row_bytes < (1LL << 31) && aligned(tokens, 16) &&
                    aligned(permute_tokens, 16);
    hipLaunchKernelGGL(mrr_route_kernel, dim3((unsigned)((A + 255) / 256)), dim3(256), 0, st, A, per_token_scales,
                       src, dst, col, (int)n_ranks, (int)n_experts, permute_scales, permute_idx);
    hipLaunchKernelGGL(mrr_copy_kernel, dim3((unsigned)((A + 3) / 4)), dim3(256), 0, st, (const uint8_t*)tokens, A,
                       row_bytes, col, (int)n_experts, (uint8_t*)permute_tokens, permute_idx, vec);
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
    TimedLaunch timed(st);
    const int sdt = scales ? scales_dtype : dtype;
    const int V = dtype == CB_DT_FLOAT32 ? 4 : 8;
    const int64_t esz = dtype == CB_DT_FLOAT32 ? 4 : 2;
    const bool vec = (H % V == 0) && K <= kMfrMaxK && H * esz < (1LL << 31) && aligned(expanded_permuted_rows, 16) &&
                     aligned(out, 16) &&
                     (!skip1 || aligned(skip1, 16)) && (!skip2 || aligned(skip2, 16)) && (!a.bias || aligned(a.bias, 16));
    const dim3 grid((unsigned)num_rows);
    const dim3 block(vec ? row_threads(H / V) : 256);
    if (!grid_fits(num_rows, block.x)) return CB_ERR_SHAPE;
#define CB_MFR(DTV, SDTV)                                                                          \
    do {                                                                                           \
        if (vec) hipLaunchKernelGGL((mfr_vec_kernel<DTV, SDTV>), grid, block, 0, st, a);           \
        else hipLaunchKernelGGL((mfr_kernel<DTV, SDTV>), grid, block, 0, st, a);                   \
    } while (0)
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
    hipStream_t st = (hipStream_t)stream;
    TimedLaunch timed(st);
    const dim3 grid((unsigned)M);
    // vector path: 16-byte rows of both halves (H a multiple of the vector width), <= 16 values per thread
    const int V = x_dtype == CB_DT_INT32 ? 4 : 8;
    const int NVcap = 16 / V;  // register budget: 16 values per thread
    if (H % V == 0 && aligned(x, 16) && aligned(y, 8) && H / V <= (int64_t)NVcap * 512) {
        const int64_t nvh = H / V;
        // kDqsqEpt values per thread (more threads per row measured faster), more for long rows
        int NVmax = (kDqsqEpt / V) < 1 ? 1 : kDqsqEpt / V;
        while (NVmax < NVcap && nvh > (int64_t)NVmax * 512) NVmax *= 2;
        // threads that cover the row in NVmax passes
        int threads = (int)(((nvh + NVmax - 1) / NVmax + 63) / 64 * 64);
        threads = threads < 64 ? 64 : threads;
        const int64_t passes = (nvh + threads - 1) / threads;
        // persistent grid: enough resident workgroups to fill every CU several times over
        const int64_t per_cu = 2048 / threads;  // waves resident per CU at this block size (occupancy 8)
        const int64_t nblk = M < 256 * per_cu * 2 ? M : 256 * per_cu * 2;
        const dim3 pgrid((unsigned)nblk);
#define CB_DQSQ_L(XDTV, NVV, QSV, LV)                                                              \
    hipLaunchKernelGGL((dqsq_vec_kernel<XDTV, NVV, QSV, LV>), pgrid, dim3(threads), 0, st, x, M, H,  \
                       weight_scale, activation_scale, quant_scale, y, scale)
#define CB_DQSQ_V(XDTV, NVV)                                                                       \
    do {                                                                                           \
        if (quant_scale && activate_left) CB_DQSQ_L(XDTV, NVV, true, true);                        \
        else if (quant_scale) CB_DQSQ_L(XDTV, NVV, true, false);                                   \
        else if (activate_left) CB_DQSQ_L(XDTV, NVV, false, true);                                 \
        else CB_DQSQ_L(XDTV, NVV, false, false);                                                   \
    } while (0)
        if (x_dtype == CB_DT_INT32) {
            if (passes <= 1) CB_DQSQ_V(CB_DT_INT32, 1);
            else if (passes <= 2) CB_DQSQ_V(CB_DT_INT32, 2);
            else CB_DQSQ_V(CB_DT_INT32, 4);
        } else if (x_dtype == CB_DT_BFLOAT16) {
            if (passes <= 1) CB_DQSQ_V(CB_DT_BFLOAT16, 1);
            else CB_DQSQ_V(CB_DT_BFLOAT16, 2);
        } else {
            if (passes <= 1) CB_DQSQ_V(CB_DT_FLOAT16, 1);
            else CB_DQSQ_V(CB_DT_FLOAT16, 2);
        }
#undef CB_DQSQ_V
#undef CB_DQSQ_L
        return check_launch();
    }
    const bool reg = H <= (int64_t)kDqsqMaxPerThread * 512;
    int threads = (int)((H + kDqsqMaxPerThread - 1) / kDqsqMaxPerThread);
    threads = (threads + 63) / 64 * 64;
    threads = threads < 64 ? 64 : (threads > 512 ? 512 : threads);
    if (!reg) threads = 512;
    if (!grid_fits(M, threads)) return CB_ERR_SHAPE;
    const dim3 block(threads);
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
    TimedLaunch timed(st);
    // E <= 256: 16 lanes per row (4 rows per wave); larger E: a whole wave per row
    const int lpr = E <= 256 ? 16 : 64;
    const int64_t rows_per_block = 4 * (64 / lpr);
    if (!grid_fits((rows + rows_per_block - 1) / rows_per_block, 256)) return CB_ERR_SHAPE;
    const dim3 grid((unsigned)((rows + rows_per_block - 1) / rows_per_block)), block(256);
    int epl = (int)((E + lpr - 1) / lpr);
    epl = epl <= 1 ? 1 : epl <= 2 ? 2 : epl <= 4 ? 4 : epl <= 8 ? 8 : epl <= 16 ? 16 : 32;
    const int vw = dtype == CB_DT_FLOAT32 ? 4 : 8;
    const bool vld = E == (int64_t)lpr * epl && epl % vw == 0 && aligned(x, 16);
#define CB_MGT(DTV, LPRV, EPLV, VLDV)                                                              \
    do {                                                                                           \
        if (k == 1)                                                                                \
            hipLaunchKernelGGL((mgt_kernel<DTV, LPRV, EPLV, VLDV, 1>), grid, block, 0, st, x, rows, (int)E, \
                               finished, (int)k, y, expert_idx, row_idx);                          \
        else if (k == 2)                                                                           \
            hipLaunchKernelGGL((mgt_kernel<DTV, LPRV, EPLV, VLDV, 2>), grid, block, 0, st, x, rows, (int)E, \
                               finished, (int)k, y, expert_idx, row_idx);                          \
        else                                                                                       \
            hipLaunchKernelGGL((mgt_kernel<DTV, LPRV, EPLV, VLDV, 4>), grid, block, 0, st, x, rows, (int)E, \
                               finished, (int)k, y, expert_idx, row_idx);                          \
    } while (0)
#define CB_MGT_V(DTV, LPRV, EPLV)                                                                  \
    do {                                                                                           \
        if constexpr (EPLV % ((DTV) == CB_DT_FLOAT32 ? 4 : 8) == 0) {                             \
            if (vld) {                                                                             \
                CB_MGT(DTV, LPRV, EPLV, true);                                                     \
                break;                                                                             \
            }                                                                                      \
        }                                                                                          \
        CB_MGT(DTV, LPRV, EPLV, false);                                                            \
    } while (0)
#define CB_MGT_E(DTV)                                                                              \
    do {                                                                                           \
        if (lpr == 16) {                                                                           \
            if (epl == 1) CB_MGT_V(DTV, 16, 1);                                                    \
            else if (epl == 2) CB_MGT_V(DTV, 16, 2);                                               \
            else if (epl == 4) CB_MGT_V(DTV, 16, 4);                                               \
            else if (epl == 8) CB_MGT_V(DTV, 16, 8);                                               \
            else CB_MGT_V(DTV, 16, 16);                                                            \
        } else {                                                                                   \
            if (epl <= 8) CB_MGT_V(DTV, 64, 8);                                                    \
            else if (epl == 16) CB_MGT_V(DTV, 64, 16);                                             \
            else CB_MGT_V(DTV, 64, 32);                                                            \
        }                                                                                          \
    } while (0)
    if (dtype == CB_DT_FLOAT32) CB_MGT_E(CB_DT_FLOAT32);
    else if (dtype == CB_DT_BFLOAT16) CB_MGT_E(CB_DT_BFLOAT16);
    else CB_MGT_E(CB_DT_FLOAT16);
#undef CB_MGT_E
#undef CB_MGT_V
#undef CB_MGT
    return check_launch();
}
