// gemm_i8.hpp - int8 x int8 -> int32 grouped GEMM: shared arguments, the skinny (decode) core and
// the generic fallback kernels for gfx950.
//
// Weights are [E, K, N] with N contiguous (the reference layout, gmsq_launch.h:62-66).  The MFMA
// B operand wants 16 consecutive K bytes per lane, so the skinny core transposes weight bytes in
// registers with v_perm_b32 (4x4 byte blocks) on their way from HBM.
//
//   skinny_kernel  decode-shaped groups (<= 16 rows per pass) of QuantMatmul and the int8 grouped
//                  down-projection (EPI_DEQUANT: the QuantMatmul dequant chain straight to bf16 /
//                  fp16) and the int32 GEMM (EPI_I32).  One workgroup = (group, 256 weight
//                  columns); its 4 waves split K, stream the weight block straight from HBM into
//                  MFMA operands (v_mfma_i32_16x16x64_i8, no LDS staging for B) and reduce their
//                  int32 partials exactly through LDS.  Weight bytes are read exactly once.
//                  GroupedMatmulSwigluQuant's decode kernel (gmsq_decode.hpp) shares its chunk
//                  load and MFMA helpers.
//   generic_*      any K / N / alignment, one thread per output (correctness path only).
// The prefill / dense LDS core is in gemm_lds.hpp, the GroupedMatmulSwigluQuant prefill kernel in
// gmsq_prefill.hpp.
#pragma once

#include "common.hpp"
#include "host_util.hpp"

namespace cb {

enum { EPI_DEQUANT = 1, EPI_I32 = 2 };

enum { BIAS_NONE = 0, BIAS_I32 = 1, BIAS_F16 = 2, BIAS_BF16 = 3, BIAS_F32 = 4 };

// Epilogue parameters.
//
// EPI_DEQUANT computes, like the reference QuantMatmul epilogue
// (quant_matmul_epilogue_kernel.cpp:15-22, 261-305):
//   v = float(c); [v += bias (int32 kind)]; v *= scale[n]; [v += offset[n]];
//   [v *= pertoken[row]]; [v += bias (float kinds)]; out = round16(v)
// scale may be offset per group (scale_gstride elements) for the grouped down-projection.
//
// GroupedMatmulSwigluQuant's epilogue computes, like the reference GMSQ vector stage
// (gmsq_vec_kernel.cpp:15-20, 207-257):
//   L = (float(c[j]) * xs[i]) * ws[g, j], R = (float(c[j+H]) * xs[i]) * ws[g, j+H]
//   act = (L / (1 + exp(-L))) * R;  amax = max |act| over the row (the bit pattern of a
//   non-negative float, combined across tiles with atomics), floored at FLT_MIN;
//   y = rint16(act * 127 / amax), y_scale = amax / 127.
struct EpiArgs {
    const void* scale;
    int64_t scale_gstride;
    int32_t scale_bf16;
    int32_t scale_perchan;
    const float* offset;
    int32_t has_offset;
    int32_t offset_perchan;
    const float* pertoken;
    int32_t has_pt;
    int32_t bias_kind;
    const void* bias;
    int32_t bias_perchan;
    int32_t out_bf16;
    int64_t bias_bstride;
    void* out;  // fp16 / bf16 for EPI_DEQUANT, int32 for EPI_I32
    int64_t out_bstride;
    // SwiGLU
    const float* w_scale;
    const float* x_scale;
    u32* amax;
    int64_t H;
    // fused requant (the persistent prefill kernel, gmsq_prefill.hpp)
    u32* arrive;       // per row tile: column tiles that have published their row maxima
    u32* status;       // set to 1 if a row tile's exchange timed out
    int8_t* yq;        // int8 output [M, H]
    float* yq_scale;   // fp32 row scales [M]
    u32* redo;         // per (row tile, column tile): the exchange wait timed out, the fix-up stores y
    int32_t spin_limit;  // polls of the exchange wait before it gives up
};

struct GemmArgs {
    const int8_t* x;
    const int8_t* w;
    int64_t M, K, N;
    int64_t x_bstride, w_bstride;  // batch strides (dense QuantMatmul)
    int64_t w_gstride;             // group stride of the weight (K * N)
    int32_t ntiles;                // tiles along N
    int32_t xcd_split;             // skinny kernel: XCDs sharing a group's column tiles (0: none)
    // Gathered activation rows (GroupedMatmulSwigluQuant with a row index): routed row r reads
    // x row row_index[r] and x_scale[row_index[r]], x holding x_rows rows.  NULL: row r is x row r.
    const int32_t* row_index;
    int64_t x_rows;
    EpiArgs epi;
    GroupTable gt;
};

// Source row of routed row r: r itself, or row_index[r]; -1 when the index lies outside
// [0, x_rows) (such a row reads as zeros with scale 0).
__device__ __forceinline__ int src_row(const GemmArgs& a, int r)
{
    if (!a.row_index) return r;
    const int s = a.row_index[r];
    return (unsigned)s < (unsigned)a.x_rows ? s : -1;
}

__device__ __forceinline__ float src_x_scale(const GemmArgs& a, int r)
{
    const int s = src_row(a, r);
    return s >= 0 ? a.epi.x_scale[s] : 0.0f;
}

__device__ __forceinline__ float load_scalar_any(const void* p, int kind, int64_t i)
{
    switch (kind) {
        case BIAS_I32: return (float)((const int32_t*)p)[i];
        case BIAS_F16: return f16_to_f32(((const uint16_t*)p)[i]);
        case BIAS_BF16: return bf16_to_f32(((const uint16_t*)p)[i]);
        default: return ((const float*)p)[i];
    }
}

// Per-column part of the dequant chain, hoisted out of the row loop.
struct ColDeq {
    float scale, offset, bias;
};

__device__ __forceinline__ ColDeq col_deq(const EpiArgs& e, int64_t g, int64_t b, int64_t col)
{
    ColDeq d;
    const int64_t si = e.scale_perchan ? col : 0;
    d.scale = e.scale_bf16 ? bf16_to_f32(((const uint16_t*)e.scale)[g * e.scale_gstride + si])
                           : ((const float*)e.scale)[g * e.scale_gstride + si];
    d.offset = e.has_offset ? e.offset[e.offset_perchan ? col : 0] : 0.0f;
    d.bias = e.bias_kind != BIAS_NONE
                 ? load_scalar_any(e.bias, e.bias_kind, b * e.bias_bstride + (e.bias_perchan ? col : 0))
                 : 0.0f;
    return d;
}

__device__ __forceinline__ float apply_deq(const EpiArgs& e, const ColDeq& d, int c, float pt)
{
    float v = (float)c;
    if (e.bias_kind == BIAS_I32) v = v + d.bias;
    v = v * d.scale;
    if (e.has_offset) v = v + d.offset;
    if (e.has_pt) v = v * pt;
    if (e.bias_kind >= BIAS_F16) v = v + d.bias;
    return v;
}

// silu(L) * R with L, R the dequantised gate / up values.  exp and the division use the hardware
// v_exp_f32 / v_rcp_f32 (about 1 ulp each), as the reference's vector unit does with its Exp and
// Div (gmsq_vec_kernel.cpp:213-218); the int8 result moves by at most one rounding step.
__device__ __forceinline__ float swiglu(float gate_c, float up_c, float xs, float wsg, float wsu)
{
    const float L = (gate_c * xs) * wsg;
    const float R = (up_c * xs) * wsu;
    return (L * __builtin_amdgcn_rcpf(1.0f + __expf(-L))) * R;
}

__device__ __forceinline__ uint4 zero4() { return make_uint4(0u, 0u, 0u, 0u); }

// Hide a value from loop-invariant code motion, so epilogue-only loads are not hoisted into
// (and kept live across) the MFMA main loop.
template <typename T>
__device__ __forceinline__ T opaque(T v)
{
    asm volatile("" : "+v"(v));
    return v;
}

// Raw buffer resource over [base, base + bytes): loads at offsets >= bytes return zeros, which
// zero-fills the K tail, and the per-lane address is one 32-bit VGPR instead of a 64-bit pointer.
constexpr int kBufFlags = 0x00020000;  // dword3 of a raw (untyped, stride 0) gfx9 buffer descriptor

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kBufFlags);
}

// Weight streams are read once: nontemporal loads (aux bit "nt") keep them from displacing the
// activations and scales in L2.
constexpr int kStreamAux = 2;
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff)
{
    const v4i v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, 0, kStreamAux);
    return make_uint4((u32)v[0], (u32)v[1], (u32)v[2], (u32)v[3]);
}

__device__ __forceinline__ uint2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t voff)
{
    typedef int v2i __attribute__((ext_vector_type(2)));
    const v2i v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, 0, 0);
    return make_uint2((u32)v[0], (u32)v[1]);
}

__device__ __forceinline__ v4i as_v4i(uint4 u)
{
    v4i r;
    r[0] = (int)u.x;
    r[1] = (int)u.y;
    r[2] = (int)u.z;
    r[3] = (int)u.w;
    return r;
}

__device__ __forceinline__ u32 comp(const uint4& v, int i)
{
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

__device__ __forceinline__ void set_comp(uint4& v, int i, u32 x)
{
    if (i == 0) v.x = x;
    else if (i == 1) v.y = x;
    else if (i == 2) v.z = x;
    else v.w = x;
}

// The activation operand of a skinny row block: a wave-uniform buffer resource and this lane's row
// offset in it (kSkOff: the row reads zeros).  A resource per lane (one per row) would make the
// compiler wrap every activation load in a readfirstlane loop over the distinct resources, and
// the wait for such a load drains every load issued before it.
constexpr uint32_t kSkOff = 0x80000000u;
struct SkinnyRow {
    __amdgpu_buffer_rsrc_t res;
    uint32_t off;   // row start of this lane (kSkOff: none)
    uint32_t k;     // row length K in bytes
};

// Row block starting at row mb of a group ending at r1; lane c takes row mb + c.  boff: the batch
// offset of x (dense QuantMatmul).  Gathered rows address all of x through the row index
// (x_rows * K < 2^31, checked on the host); contiguous rows a 16-row window from mb.
__device__ __forceinline__ SkinnyRow skinny_row(const GemmArgs& a, const int64_t boff, const int mb, const int r1,
                                                const int c)
{
    SkinnyRow s;
    const int64_t K = a.K;
    s.k = (uint32_t)K;
    const int arow = mb + c;
    if (a.row_index) {
        const int srow = arow < r1 ? src_row(a, arow) : -1;
        s.res = make_rsrc(a.x + boff, (uint32_t)(a.x_rows * K));
        s.off = srow >= 0 ? (uint32_t)srow * (uint32_t)K : kSkOff;
    } else {
        const int nrow = r1 - mb < 16 ? r1 - mb : 16;
        s.res = make_rsrc(a.x + boff + (int64_t)mb * K, (uint32_t)((int64_t)nrow * K));
        s.off = arow < r1 ? (uint32_t)c * (uint32_t)K : kSkOff;
    }
    return s;
}

// One 64-deep chunk of a skinny tile: the lane's activation operand (first, so waiting for it never
// waits for weights issued later) and 16 weight rows; k past K (and rows outside the group) read as
// zeros.
__device__ __forceinline__ void skinny_load_chunk(const SkinnyRow& xr, __amdgpu_buffer_rsrc_t wres,
                                                  const uint32_t lane_off, const uint32_t n, const int q,
                                                  const int kc, uint4 (&R)[16], v4i& A)
{
    const uint32_t k = (uint32_t)(kc * 64 + q * 16);
    A = __builtin_amdgcn_raw_buffer_load_b128(xr.res, xr.off != kSkOff && k < xr.k ? xr.off + k : kSkOff, 0, 0);
    const uint32_t kofs = (uint32_t)(kc * 64) * n;
#pragma unroll
    for (int i = 0; i < 16; ++i) R[i] = buf_load16(wres, lane_off + kofs + (uint32_t)i * n);
}

// The chunk's MFMAs: the 16 loaded rows are transposed in registers into 16 B operands, one per
// column, and MFMA j accumulates column 16 c + j.
__device__ __forceinline__ void skinny_mma_chunk(const uint4 (&R)[16], const v4i av, v4i (&acc)[16])
{
    // column block cb: the 4 B operands of columns 4 cb .. 4 cb + 3, built from dword cb of the 16
    // loaded rows, consumed right away to keep the live range short
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        uint4 T[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            u32 o0, o1, o2, o3;
            transpose4x4_b8(comp(R[4 * rb + 0], cb), comp(R[4 * rb + 1], cb), comp(R[4 * rb + 2], cb),
                            comp(R[4 * rb + 3], cb), o0, o1, o2, o3);
            set_comp(T[0], rb, o0);
            set_comp(T[1], rb, o1);
            set_comp(T[2], rb, o2);
            set_comp(T[3], rb, o3);
        }
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4)
            acc[4 * cb + s4] = __builtin_amdgcn_mfma_i32_16x16x64_i8(av, as_v4i(T[s4]), acc[4 * cb + s4], 0, 0, 0);
    }
}

// Epilogue of one output row of a skinny tile: lane (q, c) holds s[j] = C[row][ocol + j] (SwiGLU:
// gate columns in lanes c < 8, their up partners 8 lanes away).  Every lane of the wave calls it.
template <int EPI>
__device__ __forceinline__ void skinny_row_epilogue(const GemmArgs& a, const int g, const int64_t b, const int row,
                                                    const bool rowok, const bool colok, const int64_t ocol,
                                                    const int64_t col, const int c, const int (&s)[16])
{
    const int64_t N = a.N;
    const EpiArgs& e = a.epi;
    (void)col;
    if constexpr (EPI == EPI_I32) {
        if (rowok && colok) {
            int4* dst = reinterpret_cast<int4*>((int32_t*)e.out + b * e.out_bstride + (int64_t)row * N + ocol);
#pragma unroll
            for (int j = 0; j < 4; ++j) dst[j] = make_int4(s[4 * j], s[4 * j + 1], s[4 * j + 2], s[4 * j + 3]);
        }
    } else {
        if (rowok && colok) {
            const float pt = e.has_pt ? e.pertoken[row] : 1.0f;
            const int64_t oc = opaque(ocol);
            u32 packed[8];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float v = apply_deq(e, col_deq(e, g, b, oc + j), s[j], pt);
                const u32 h = e.out_bf16 ? f32_to_bf16(v) : f32_to_f16(v);
                packed[j / 2] = (j & 1) ? (packed[j / 2] | (h << 16)) : h;
            }
            uint4* dst = reinterpret_cast<uint4*>((uint16_t*)e.out + b * e.out_bstride + (int64_t)row * N + ocol);
            dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
            dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
        }
    }
}

// Block -> (group, column tile) of the skinny kernels.  a.xcd_split = P > 0: XCD pair / quad p
// streams groups p, p + 8 / P, ... and each of its P XCDs one contiguous 1 / P of their column
// tiles (workgroups are dispatched round-robin over the 8 XCDs in linear block order).
__device__ __forceinline__ void skinny_block(const GemmArgs& a, int& g, int& ct)
{
    g = blockIdx.y;
    ct = blockIdx.x;
    const int P = a.xcd_split;
    if (P > 0) {
        const int G = 8 / P;
        const int lin = blockIdx.y * gridDim.x + blockIdx.x;
        const int x = lin & 7, j = lin >> 3, h = gridDim.x / P;
        g = (j / h) * G + x / P;
        ct = (x % P) * h + j % h;
    }
}

// ============================================================================================
// skinny_kernel: decode-shaped groups.
//   grid = (ntiles, E), block = 256 (4 waves).  SwiGLU tiles cover 128 gate + 128 up columns,
//   dequant tiles cover 256 columns.  Lane l of every wave owns k-group q = l / 16 and column
//   group c = l % 16 (16 consecutive weight columns); after the in-register 16x16 byte transpose
//   the lane holds 16 B operands, one per column, and MFMA j yields column (16 c + j).
// ============================================================================================
template <int EPI>
__global__ __launch_bounds__(256, 2) void skinny_kernel(const GemmArgs a)
{
    __shared__ int red[3][4][16][64];  // partial sums handed to the wave that owns them (48 KiB)

    // Block -> (group, column tile).  Workgroups are dispatched round-robin over the 8 XCDs in
    // linear block order; remapped, XCD pair p streams groups p, p + 4, ... and each XCD of the
    // pair one contiguous half of their column tiles, i.e. every XCD reads one contiguous 2 KB
    // (16 column tiles) or 3.5 KB (28) run of each weight row instead of two scattered 256-byte
    // pieces.  Measured on a weight-streaming probe: 6.3 vs 5.5 TB/s.  Needs an even tile count
    // and a group count divisible by 4 (the host passes the grid as is otherwise).
    int g, ct;
    skinny_block(a, g, ct);
    const int r0 = g ? a.gt.row_end[g - 1] : 0;
    const int r1 = a.gt.row_end[g];
    if (r0 >= r1) return;

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4, c = lane & 15;
    const int64_t K = a.K, N = a.N;

    const int64_t ocol = (int64_t)ct * 256 + 16 * c;  // first weight / output column of this lane
    const bool colok = ocol < N;
    const int64_t col = ocol;
    const int64_t b = blockIdx.z;  // batch (dense QuantMatmul)
    // weight block of this group (the host sends K * N >= 2^31 to the generic kernels)
    const __amdgpu_buffer_rsrc_t wres = make_rsrc(a.w + b * a.w_bstride + (int64_t)g * a.w_gstride, (uint32_t)(K * N));
    const uint32_t lane_off = (uint32_t)(colok ? col : 0) + (uint32_t)(q * 16) * (uint32_t)N;
    const int nch = (int)((K + 63) >> 6);

    for (int mb = r0; mb < r1; mb += 16) {
        v4i acc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = v4i{0, 0, 0, 0};

        // activation row of this lane: rows past the group (or gathered from outside x) and k past
        // K read as zeros without a branch, so the activation load joins its chunk's weight loads
        const SkinnyRow xres = skinny_row(a, b * a.x_bstride, mb, r1, c);

        // one chunk = the activation operand (first, so waiting for it never waits for weights
        // issued later) and 16 weight rows
        auto load_chunk = [&](int kc, uint4 (&R)[16], v4i& A) {
            skinny_load_chunk(xres, wres, lane_off, (uint32_t)N, q, kc, R, A);
        };
        auto mma_chunk = [&](const uint4 (&R)[16], const v4i av) { skinny_mma_chunk(R, av, acc); };

        for (int kc = wave; kc < nch; kc += 4) {
            uint4 R[16];
            v4i A;
            load_chunk(kc, R, A);
            mma_chunk(R, A);
        }

        // Cross-wave K reduction: wave w keeps accumulator row r == w and receives the other
        // three waves' partials for it through LDS.
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (r != wave) {
                const int slot = wave < r ? wave : wave - 1;
#pragma unroll
                for (int j = 0; j < 16; ++j) red[slot][r][j][lane] = acc[j][r];
            }
        }
        __syncthreads();
        int s[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            int v = 0;
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (r == wave) v = acc[j][r];
            s[j] = v + red[0][wave][j][lane] + red[1][wave][j][lane] + red[2][wave][j][lane];
        }
        __syncthreads();  // the next row block reuses red[]

        // MFMA 16x16 C layout: lane l holds rows 4 (l / 16) + r, column l % 16.
        const int row = mb + 4 * q + wave;
        skinny_row_epilogue<EPI>(a, g, b, row, row < r1, colok, ocol, col, c, s);
    }
}

// Group of row tile mt in a GroupTable enumeration.
__device__ __forceinline__ int group_of_tile(const GroupTable& gt, int mt)
{
    int lo = 0, hi = gt.n_groups - 1;
    while (lo < hi) {  // last g with tile_start[g] <= mt and a non-empty tile range
        const int mid = (lo + hi + 1) >> 1;
        if (gt.tile_start[mid] <= mt) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// ============================================================================================
// generic kernels: any K / N / alignment.  One thread per output, byte loads.  Used only for
// shapes the vector paths do not cover (K % 16 != 0, N % 32 != 0, unaligned pointers).
// ============================================================================================
__device__ __forceinline__ int group_of_row(const GroupTable& gt, int row)
{
    int lo = 0, hi = gt.n_groups - 1;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (gt.row_end[mid] > row) hi = mid;
        else lo = mid + 1;
    }
    return lo;
}

// The generic kernels walk virtual blocks vb = (row, 256-column tile) with a grid-stride loop, so
// any M x tiles count fits a launch (a dispatch counts its work-items in 32 bits).
// GroupedMatmulSwigluQuant for shapes off the vector paths, in two passes over the same products
// (no intermediate in memory): QUANT = false publishes the per-row |act| maxima, QUANT = true
// recomputes act and writes y = rint16(act * 127 / amax) and y_scale (column tile 0, thread 0).
template <bool QUANT>
static __global__ __launch_bounds__(256) void generic_swiglu_kernel(const GemmArgs a)
{
    const int64_t H = a.epi.H;
    const int64_t nvb = a.M * a.ntiles;
    for (int64_t vb = blockIdx.x; vb < nvb; vb += gridDim.x) {
        const int row = (int)(vb / a.ntiles);
        const int64_t idx = (vb % a.ntiles) * 256 + threadIdx.x;
        const bool ok = idx < H;
        const int g = group_of_row(a.gt, row);
        float v = 0.0f;
        if (ok) {
            const int srow = src_row(a, row);
            const int8_t* xr = a.x + (int64_t)(srow >= 0 ? srow : 0) * a.K;
            const int8_t* wg = a.w + (int64_t)g * a.w_gstride;
            int cg = 0, cu = 0;
            for (int64_t k = 0; k < a.K; ++k) {
                const int xv = srow >= 0 ? xr[k] : 0;
                cg += xv * (int)wg[k * a.N + idx];
                cu += xv * (int)wg[k * a.N + H + idx];
            }
            v = swiglu((float)cg, (float)cu, src_x_scale(a, row), a.epi.w_scale[(int64_t)g * a.N + idx],
                       a.epi.w_scale[(int64_t)g * a.N + H + idx]);
        }
        if constexpr (!QUANT) {
            const float m = wave_max(ok ? fabsf(v) : 0.0f);
            if ((threadIdx.x & 63) == 0) atomicMax(a.epi.amax + row, __float_as_uint(m));
        } else {
            float am = __uint_as_float(a.epi.amax[row]);
            if (!(am > kFltMin)) am = kFltMin;
            if (ok) a.epi.yq[(int64_t)row * H + idx] = (int8_t)rint16(v * (127.0f / am));
            if (vb % a.ntiles == 0 && threadIdx.x == 0) a.epi.yq_scale[row] = am * kInv127;
        }
    }
}

static __global__ __launch_bounds__(256) void generic_dequant_kernel(const GemmArgs a)
{
    const int64_t b = blockIdx.y;
    const int64_t nvb = a.M * a.ntiles;
    const EpiArgs& e = a.epi;
    for (int64_t vb = blockIdx.x; vb < nvb; vb += gridDim.x) {
        const int row = (int)(vb / a.ntiles);
        const int64_t col = (vb % a.ntiles) * 256 + threadIdx.x;
        if (col >= a.N) continue;
        const int g = group_of_row(a.gt, row);
        const int8_t* xr = a.x + b * a.x_bstride + (int64_t)row * a.K;
        const int8_t* wg = a.w + b * a.w_bstride + (int64_t)g * a.w_gstride;
        int acc = 0;
        for (int64_t k = 0; k < a.K; ++k) acc += (int)xr[k] * (int)wg[k * a.N + col];
        const ColDeq d = col_deq(e, g, b, col);
        const float pt = e.has_pt ? e.pertoken[row] : 1.0f;
        const float v = apply_deq(e, d, acc, pt);
        uint16_t* ob = (uint16_t*)e.out + b * e.out_bstride;
        ob[(int64_t)row * a.N + col] = e.out_bf16 ? f32_to_bf16(v) : f32_to_f16(v);
    }
}

static __global__ __launch_bounds__(256) void generic_i32_kernel(const GemmArgs a)
{
    const int64_t b = blockIdx.y;
    const int64_t nvb = a.M * a.ntiles;
    for (int64_t vb = blockIdx.x; vb < nvb; vb += gridDim.x) {
        const int row = (int)(vb / a.ntiles);
        const int64_t col = (vb % a.ntiles) * 256 + threadIdx.x;
        if (col >= a.N) continue;
        const int g = group_of_row(a.gt, row);
        const int8_t* xr = a.x + b * a.x_bstride + (int64_t)row * a.K;
        const int8_t* wg = a.w + b * a.w_bstride + (int64_t)g * a.w_gstride;
        int acc = 0;
        for (int64_t k = 0; k < a.K; ++k) acc += (int)xr[k] * (int)wg[k * a.N + col];
        ((int32_t*)a.epi.out + b * a.epi.out_bstride)[(int64_t)row * a.N + col] = acc;
    }
}

}  // namespace cb
