// norm_quant.hip - AddRmsNormDynamicQuant and DynamicQuant for gfx950.
//
// Both operators are HBM-streaming row kernels: one workgroup owns one row, each thread keeps its
// slice of the row in registers, so the inputs are read from HBM exactly once and every output is
// written exactly once.  The per-row sum of squares and abs-max are wave64 shuffle reductions
// followed by a cross-wave reduction through LDS.
//
// Semantics (reference):
//   ARDQ  operators/addrmsnormdynamicquant/csrc/ops/add_rms_norm_dynamic_quant/op_kernel/
//         add_rms_norm_dynamic_quant_kernel.cpp:15-30 (algebra), 440-503 (per-row order of operations)
//   DQ    operators/dynamicquant/csrc/ops/dynamic_quant/op_kernel/dynamic_quant_kernel.cpp:15-26,240-282
#include <climits>

#include "common.hpp"
#include "host_util.hpp"

namespace cb {

constexpr int kRowMaxWaves = 8;

// Reduce (sum, max) across the workgroup.  Every thread gets both results.
__device__ __forceinline__ void block_sum_max(float& s, float& m, float* red)
{
    s = wave_sum(s);
    m = wave_max(m);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    if (lane == 0) {
        red[wave] = s;
        red[kRowMaxWaves + wave] = m;
    }
    __syncthreads();
    s = 0.0f;
    m = 0.0f;
    for (int w = 0; w < nw; ++w) {
        s += red[w];
        m = fmaxf(m, red[kRowMaxWaves + w]);
    }
}

// Row slice owned by a thread: NV vectors of VEC elements at element offset ((i*blockDim)+tid)*VEC.
template <int VEC>
struct Vec16 {
    uint16_t v[VEC];
};

typedef int rv4i __attribute__((ext_vector_type(4)));

template <int VEC>
__device__ __forceinline__ Vec16<VEC> ldv(const uint16_t* p)
{
    Vec16<VEC> r;
    if constexpr (VEC == 8) {
        // row data is read exactly once: nontemporal loads keep it from displacing other lines
        const rv4i q = __builtin_nontemporal_load(reinterpret_cast<const rv4i*>(p));
        __builtin_memcpy(r.v, &q, 16);
    } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) r.v[j] = p[j];
    }
    return r;
}

template <int VEC>
__device__ __forceinline__ void stv(uint16_t* p, const Vec16<VEC>& r)
{
    if constexpr (VEC == 8) {
        rv4i q;
        __builtin_memcpy(&q, r.v, 16);
        __builtin_nontemporal_store(q, reinterpret_cast<rv4i*>(p));
    } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) p[j] = r.v[j];
    }
}

template <int VEC>
__device__ __forceinline__ void sty8(int8_t* p, const int* q)
{
    if constexpr (VEC == 8) {
        typedef int rv2i __attribute__((ext_vector_type(2)));
        rv2i w;
        w[0] = (int)pack4_i8(q[0], q[1], q[2], q[3]);
        w[1] = (int)pack4_i8(q[4], q[5], q[6], q[7]);
        __builtin_nontemporal_store(w, reinterpret_cast<rv2i*>(p));
    } else {
#pragma unroll
        for (int j = 0; j < VEC; ++j) p[j] = (int8_t)q[j];
    }
}

// AddRmsNormDynamicQuant: one workgroup per row.
template <bool BF16, int VEC, int NV>
__global__ __launch_bounds__(512) void ardq_kernel(const uint16_t* __restrict__ x1,
                                                   const uint16_t* __restrict__ x2,
                                                   const uint16_t* __restrict__ gamma,
                                                   int64_t n, float eps, float invN,
                                                   int8_t* __restrict__ y, uint16_t* __restrict__ xout,
                                                   float* __restrict__ scale)
{
    __shared__ float red[2 * kRowMaxWaves];
    const int64_t row = blockIdx.x;
    const int64_t base = row * n;
    const int nvec = (int)(n / VEC);
    float z[NV][VEC];
    float ss = 0.0f, mz = 0.0f;
    if constexpr (VEC == 8) {
        // 16-byte rows through buffer resources: every load of the thread's slice is issued up
        // front with no branch (lanes past the row read zeros, which add nothing to the sums, and
        // their stores are dropped), so the whole slice is in flight at once
        const uint32_t rb = (uint32_t)(n * 2);
        const auto r1 = row_rsrc(x1 + base, rb), r2 = row_rsrc(x2 + base, rb), rg = row_rsrc(gamma, rb);
        const auto ro = row_rsrc(xout + base, rb);
        uint32_t off[NV];
        v4i A[NV], B[NV], G[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = i * blockDim.x + threadIdx.x;
            off[i] = v < nvec ? (uint32_t)v * 16u : kOffNone;
            A[i] = row_load(r1, off[i]);
            B[i] = row_load(r2, off[i]);
            G[i] = __builtin_amdgcn_raw_buffer_load_b128(rg, off[i], 0, 0);  // gamma is shared by all rows
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint16_t* a = reinterpret_cast<const uint16_t*>(&A[i]);
            const uint16_t* b = reinterpret_cast<const uint16_t*>(&B[i]);
            const uint16_t* g = reinterpret_cast<const uint16_t*>(&G[i]);
            uint16_t o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float xf = ld16<BF16>(a[j]) + ld16<BF16>(b[j]);
                o[j] = st16<BF16>(xf);
                ss += xf * xf;
                z[i][j] = xf * ld16<BF16>(g[j]);
                mz = fmaxf(mz, fabsf(z[i][j]));
            }
            v4i ov;
            __builtin_memcpy(&ov, o, 16);
            row_store(ov, ro, off[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = i * blockDim.x + threadIdx.x;
            if (v < nvec) {
                const int64_t e = base + (int64_t)v * VEC;
                Vec16<VEC> a = ldv<VEC>(x1 + e), b = ldv<VEC>(x2 + e), g = ldv<VEC>(gamma + (int64_t)v * VEC);
                Vec16<VEC> o;
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    const float xf = ld16<BF16>(a.v[j]) + ld16<BF16>(b.v[j]);
                    o.v[j] = st16<BF16>(xf);
                    ss += xf * xf;
                    z[i][j] = xf * ld16<BF16>(g.v[j]);
                    mz = fmaxf(mz, fabsf(z[i][j]));
                }
                stv<VEC>(xout + e, o);
            }
        }
    }
    block_sum_max(ss, mz, red);
    const float rms = sqrtf(ss * invN + eps);
    const float rstd = 1.0f / rms;
    const float m = mz * rstd;
    const float sm = (m < 1e-12f) ? 1e-12f : m;  // NaN passes through like the reference
    const float sc = sm * kInv127;
    const float k = rstd / sc;
    if (threadIdx.x == 0) scale[row] = sc;
    if constexpr (VEC == 8) {
        const auto ry = row_rsrc(y + base, (uint32_t)n);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = i * blockDim.x + threadIdx.x;
            int q[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) q[j] = rint16(z[i][j] * k);
            typedef int rv2i __attribute__((ext_vector_type(2)));
            rv2i w;
            w[0] = (int)pack4_i8(q[0], q[1], q[2], q[3]);
            w[1] = (int)pack4_i8(q[4], q[5], q[6], q[7]);
            __builtin_amdgcn_raw_buffer_store_b64(w, ry, v < nvec ? (uint32_t)v * 8u : kOffNone, 0, 2);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = i * blockDim.x + threadIdx.x;
            if (v < nvec) {
                int q[VEC];
#pragma unroll
                for (int j = 0; j < VEC; ++j) q[j] = rint16(z[i][j] * k);
                sty8<VEC>(y + base + (int64_t)v * VEC, q);
            }
        }
    }
}

// DynamicQuant: one workgroup per row.
template <bool BF16, int VEC, int NV>
__global__ __launch_bounds__(512) void dq_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                 int8_t* __restrict__ y, float* __restrict__ scale)
{
    __shared__ float red[2 * kRowMaxWaves];
    const int64_t base = (int64_t)blockIdx.x * n;
    const int nvec = (int)(n / VEC);
    float xv[NV][VEC];
    float s = 0.0f, a = 0.0f;
    if constexpr (VEC == 8) {
        // branch-free 16-byte buffer loads of the whole slice (zeros past the row)
        const auto rx = row_rsrc(x + base, (uint32_t)(n * 2));
        v4i X[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = i * blockDim.x + threadIdx.x;
            X[i] = row_load(rx, v < nvec ? (uint32_t)v * 16u : kOffNone);
        }
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const uint16_t* t = reinterpret_cast<const uint16_t*>(&X[i]);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                xv[i][j] = ld16<BF16>(t[j]);
                a = fmaxf(a, fabsf(xv[i][j]));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int v = i * blockDim.x + threadIdx.x;
            if (v < nvec) {
                Vec16<VEC> t = ldv<VEC>(x + base + (int64_t)v * VEC);
#pragma unroll
                for (int j = 0; j < VEC; ++j) {
                    xv[i][j] = ld16<BF16>(t.v[j]);
                    a = fmaxf(a, fabsf(xv[i][j]));
                }
            }
        }
    }
    block_sum_max(s, a, red);
    a = fmaxf(a, 1e-12f);
    if (threadIdx.x == 0) scale[blockIdx.x] = a * kInv127;
    const float inv = 127.0f * (1.0f / a);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int v = i * blockDim.x + threadIdx.x;
        if (v < nvec) {
            int q[VEC];
#pragma unroll
            for (int j = 0; j < VEC; ++j) q[j] = rint16(xv[i][j] * inv);
            sty8<VEC>(y + base + (int64_t)v * VEC, q);
        }
    }
}

// DynamicQuant for rows longer than one workgroup's register slice: two passes over the row
// (abs-max, then quantise), the second one served mostly from L2.
template <bool BF16>
__global__ __launch_bounds__(512) void dq_long_kernel(const uint16_t* __restrict__ x, int64_t n,
                                                      int8_t* __restrict__ y, float* __restrict__ scale)
{
    __shared__ float red[2 * kRowMaxWaves];
    const uint16_t* xr = x + (int64_t)blockIdx.x * n;
    int8_t* yr = y + (int64_t)blockIdx.x * n;
    float s = 0.0f, a = 0.0f;
    for (int64_t j = threadIdx.x; j < n; j += blockDim.x) a = fmaxf(a, fabsf(ld16<BF16>(xr[j])));
    block_sum_max(s, a, red);
    a = fmaxf(a, 1e-12f);
    if (threadIdx.x == 0) scale[blockIdx.x] = a * kInv127;
    const float inv = 127.0f * (1.0f / a);
    for (int64_t j = threadIdx.x; j < n; j += blockDim.x) yr[j] = (int8_t)rint16(ld16<BF16>(xr[j]) * inv);
}

// ---------------------------------------------------------------------------------------------
// Host side: pick (VEC, threads, NV) and launch.
// ---------------------------------------------------------------------------------------------
struct RowPlan {
    int vec;
    int threads;
    int nv;
};

constexpr int kRowMaxThreads = 512;

// Row split: VEC elements per access (8 when rows are 16-byte aligned), `threads` a multiple of 64,
// NV accesses per thread.  Vector path: the (threads, NV <= 8) pair with the fewest idle slots,
// preferring wider workgroups up to kRowMaxThreads.  Scalar path: powers of two.
static RowPlan plan_row(int64_t n, bool aligned16)
{
    RowPlan p;
    p.vec = (aligned16 && n % 8 == 0) ? 8 : 1;
    const int64_t nvec = n / p.vec;
    if (p.vec == 8) {
        int best_t = 64, best_nv = 8;
        int64_t best_waste = INT64_MAX;
        for (int t = 64; t <= 512; t += 64) {
            const int64_t nv = (nvec + t - 1) / t;
            if (nv > 8) continue;
            const int64_t waste = t * nv - nvec;
            const bool better = waste < best_waste ||
                                (waste == best_waste && t <= kRowMaxThreads && (best_t > kRowMaxThreads || t > best_t));
            if (better) {
                best_waste = waste;
                best_t = t;
                best_nv = (int)nv;
            }
        }
        p.threads = best_t;
        p.nv = best_nv;
        return p;
    }
    int64_t t = (nvec + 63) / 64 * 64;
    p.threads = (int)(t < 64 ? 64 : (t > 256 ? 256 : t));
    int64_t need = (nvec + p.threads - 1) / p.threads;
    int nv = 1;
    while (nv < need) nv <<= 1;
    if (nv > 32) {  // keep the register slice bounded: widen the workgroup instead
        p.threads = 512;
        need = (nvec + 511) / 512;
        nv = 1;
        while (nv < need) nv <<= 1;
    }
    p.nv = nv;
    return p;
}

template <bool BF16, int VEC>
static hipError_t launch_ardq_v(const RowPlan& p, int64_t rows, const uint16_t* x1, const uint16_t* x2,
                                const uint16_t* g, int64_t n, float eps, float invN, int8_t* y,
                                uint16_t* xo, float* sc, hipStream_t st)
{
    dim3 grid((unsigned)rows), block(p.threads);
#define CB_ARDQ_CASE(NVV)                                                                          \
    case NVV:                                                                                      \
        hipLaunchKernelGGL((ardq_kernel<BF16, VEC, NVV>), grid, block, 0, st, x1, x2, g, n, eps,   \
                           invN, y, xo, sc);                                                       \
        break;
    if constexpr (VEC == 8) {
        switch (p.nv) {
            CB_ARDQ_CASE(1)
            CB_ARDQ_CASE(2)
            CB_ARDQ_CASE(3)
            CB_ARDQ_CASE(4)
            CB_ARDQ_CASE(5)
            CB_ARDQ_CASE(6)
            CB_ARDQ_CASE(7)
            CB_ARDQ_CASE(8)
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (p.nv) {
            CB_ARDQ_CASE(1)
            CB_ARDQ_CASE(2)
            CB_ARDQ_CASE(4)
            CB_ARDQ_CASE(8)
            CB_ARDQ_CASE(16)
            CB_ARDQ_CASE(32)
            default: return hipErrorInvalidValue;
        }
    }
#undef CB_ARDQ_CASE
    return hipGetLastError();
}

template <bool BF16, int VEC>
static hipError_t launch_dq_v(const RowPlan& p, int64_t rows, const uint16_t* x, int64_t n, int8_t* y,
                              float* sc, hipStream_t st)
{
    dim3 grid((unsigned)rows), block(p.threads);
#define CB_DQ_CASE(NVV)                                                                            \
    case NVV:                                                                                      \
        hipLaunchKernelGGL((dq_kernel<BF16, VEC, NVV>), grid, block, 0, st, x, n, y, sc);          \
        break;
    if constexpr (VEC == 8) {
        switch (p.nv) {
            CB_DQ_CASE(1)
            CB_DQ_CASE(2)
            CB_DQ_CASE(3)
            CB_DQ_CASE(4)
            CB_DQ_CASE(5)
            CB_DQ_CASE(6)
            CB_DQ_CASE(7)
            CB_DQ_CASE(8)
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (p.nv) {
            CB_DQ_CASE(1)
            CB_DQ_CASE(2)
            CB_DQ_CASE(4)
            CB_DQ_CASE(8)
            CB_DQ_CASE(16)
            CB_DQ_CASE(32)
            default: return hipErrorInvalidValue;
        }
    }
#undef CB_DQ_CASE
    return hipGetLastError();
}

}  // namespace cb

using namespace cb;

extern "C" int cb_add_rms_norm_dynamic_quant(const void* x1, const void* x2, const void* gamma, int dtype,
                                             int64_t rows, int64_t row_len, float epsilon, int8_t* y,
                                             void* x_out, float* scale_out, void* stream)
{
    if (dtype != CB_DT_FLOAT16 && dtype != CB_DT_BFLOAT16) return CB_ERR_DTYPE;
    if (rows < 0 || row_len < 0) return CB_ERR_SHAPE;
    if (rows == 0 || row_len == 0) return CB_OK;
    if (row_len > CB_ARDQ_MAX_ROW) return CB_ERR_ROW_TOO_LONG;
    if (rows > 0x7fffffffLL) return CB_ERR_SHAPE;
    if (!x1 || !x2 || !gamma || !y || !x_out || !scale_out) return CB_ERR_NULL_POINTER;
    const bool al = aligned(x1, 16) && aligned(x2, 16) && aligned(gamma, 16) && aligned(x_out, 16) &&
                    aligned(y, 8);
    RowPlan p = plan_row(row_len, al);
    if (!grid_fits(rows, p.threads)) return CB_ERR_SHAPE;
    const float invN = 1.0f / (float)row_len;
    hipStream_t st = (hipStream_t)stream;
    TimedLaunch timed(st);
    auto a = (const uint16_t*)x1;
    auto b = (const uint16_t*)x2;
    auto g = (const uint16_t*)gamma;
    auto xo = (uint16_t*)x_out;
    hipError_t e;
    if (dtype == CB_DT_BFLOAT16)
        e = (p.vec == 8) ? launch_ardq_v<true, 8>(p, rows, a, b, g, row_len, epsilon, invN, y, xo, scale_out, st)
                         : launch_ardq_v<true, 1>(p, rows, a, b, g, row_len, epsilon, invN, y, xo, scale_out, st);
    else
        e = (p.vec == 8) ? launch_ardq_v<false, 8>(p, rows, a, b, g, row_len, epsilon, invN, y, xo, scale_out, st)
                         : launch_ardq_v<false, 1>(p, rows, a, b, g, row_len, epsilon, invN, y, xo, scale_out, st);
    return e == hipSuccess ? CB_OK : CB_ERR_LAUNCH;
}

extern "C" int cb_dynamic_quant(const void* x, int dtype, int64_t rows, int64_t row_len, int8_t* y,
                                float* scale, void* stream)
{
    if (dtype != CB_DT_FLOAT16 && dtype != CB_DT_BFLOAT16) return CB_ERR_DTYPE;
    if (rows < 0 || row_len < 0) return CB_ERR_SHAPE;
    if (row_len == 0) return CB_ERR_EMPTY;  // the reference requires a non-zero last dimension
    if (rows == 0) return CB_OK;
    if (rows > 0x7fffffffLL) return CB_ERR_SHAPE;
    if (!x || !y || !scale) return CB_ERR_NULL_POINTER;
    if (!grid_fits(rows, 512)) return CB_ERR_SHAPE;  // the widest block any path below uses
    hipStream_t st = (hipStream_t)stream;
    TimedLaunch timed(st);
    if (row_len > 16384) {  // longer than a register-resident row slice
        if (dtype == CB_DT_BFLOAT16)
            hipLaunchKernelGGL(dq_long_kernel<true>, dim3((unsigned)rows), dim3(512), 0, st, (const uint16_t*)x, row_len, y, scale);
        else
            hipLaunchKernelGGL(dq_long_kernel<false>, dim3((unsigned)rows), dim3(512), 0, st, (const uint16_t*)x, row_len, y, scale);
        return hipGetLastError() == hipSuccess ? CB_OK : CB_ERR_LAUNCH;
    }
    RowPlan p = plan_row(row_len, aligned(x, 16) && aligned(y, 8));
    auto xp = (const uint16_t*)x;
    hipError_t e;
    if (dtype == CB_DT_BFLOAT16)
        e = (p.vec == 8) ? launch_dq_v<true, 8>(p, rows, xp, row_len, y, scale, st)
                         : launch_dq_v<true, 1>(p, rows, xp, row_len, y, scale, st);
    else
        e = (p.vec == 8) ? launch_dq_v<false, 8>(p, rows, xp, row_len, y, scale, st)
                         : launch_dq_v<false, 1>(p, rows, xp, row_len, y, scale, st);
    return e == hipSuccess ? CB_OK : CB_ERR_LAUNCH;
}
