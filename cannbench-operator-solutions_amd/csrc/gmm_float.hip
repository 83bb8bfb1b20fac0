// gmm_float.hip - GroupedMatmul, the reference's float grouped GEMM (C ABI cb_grouped_matmul):
//   y[rows_g] = x[rows_g] @ weight[g] (+ bias[g]),  rows_g = [group_list[g-1], group_list[g])
// in the dtype of x (fp16, bf16 or fp32), weight [E, K, N] or, with transpose_weight, [E, N, K]
// (operators/groupedmatmul/csrc/ops/grouped_matmul/op_plugin/grouped_matmul_plugin.cpp:14-17,
// 116-183; op_kernel/grouped_matmul_kernel.cpp:15-17, 111-150).
//
// 16-bit inputs run on v_mfma_f32_32x32x16_{f16,bf16}: 128 x 128 output tiles (4 waves of 64 x 64),
// 32-deep K stages double-buffered in LDS with both operands stored K-contiguous (the weight is
// transposed on its way into LDS when it arrives N-contiguous), fp32 accumulation, the bias added
// in fp32, one round-to-nearest-even narrowing.  fp32 inputs and shapes off the vector path
// (K or N not a multiple of 8, misaligned operands, 32-bit offsets exceeded) take a plain fp32 loop.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <set>
#include <utility>

#include "gemm_lds.hpp"

namespace cb {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short v4i16 __attribute__((ext_vector_type(4)));

constexpr int kGmmMaxExperts = 64;  // GMM_MAX_E (grouped_matmul_launch.h)
constexpr int GF_BK = 32;
// elements per LDS row (BK + 8: 80 B at BK 32): a 16-lane b128 read phase hits 16 distinct bank groups
constexpr int GF_PITCH = GF_BK + 8;
constexpr int GF_KCH = GF_BK / 8;  // 16-byte chunks per row and stage

struct GmmFArgs {
    const void* x;
    const void* w;
    const void* bias;
    void* y;
    int64_t M, K, N;
    int32_t x_dt, bias_dt;  // cb_dtype codes; bias_dt 0 = no bias
    int32_t trans, ntiles;
    GroupTable gt;
};

__device__ __forceinline__ float gf_load(const void* p, int dt, int64_t i)
{
    if (dt == CB_DT_FLOAT32) return ((const float*)p)[i];
    if (dt == CB_DT_BFLOAT16) return bf16_to_f32(((const uint16_t*)p)[i]);
    return f16_to_f32(((const uint16_t*)p)[i]);
}

__device__ __forceinline__ void gf_store(void* p, int dt, int64_t i, float v)
{
    if (dt == CB_DT_FLOAT32) ((float*)p)[i] = v;
    else if (dt == CB_DT_BFLOAT16) ((uint16_t*)p)[i] = f32_to_bf16_hw(v);
    else ((uint16_t*)p)[i] = f32_to_f16(v);
}

// One BM x BN tile per workgroup of WM x WN waves (wave tiles (BM / WM) x (BN / WN)): pid -> (row
// tile, column tile) with 4 row tiles per column sweep.  Launched as 128 x 128 with 2 x 2 waves.
template <bool BF16, bool TRANS, int GF_BM, int GF_BN, int WM, int WN>
__global__ __launch_bounds__(64 * WM * WN, 64 * WM * WN > 256 ? 1 : 2) void gmm_mfma_kernel(const GmmFArgs a)
{
    constexpr int NT = 64 * WM * WN;
    constexpr int TM = GF_BM / WM, TN = GF_BN / WN, FM = TM / 32, FN = TN / 32;
    constexpr int GF_CA = GF_BM * GF_KCH / NT;             // A chunks per thread
    constexpr int GF_CB = GF_BN * GF_KCH / NT;             // [N][K] weight chunks per thread
    constexpr int GF_CP = (GF_BK / 2) * (GF_BN / 8) / NT;  // [K][N] weight: (k, k + 1) chunk pairs per thread
    constexpr int NCH = GF_BN / 8;                         // 8-column chunks per weight row
    static_assert(GF_CA >= 1 && GF_CB >= 1 && GF_CP >= 1, "tile too small for the workgroup");
    __shared__ __attribute__((aligned(16))) uint16_t As[2][GF_BM * GF_PITCH];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][GF_BN * GF_PITCH];  // [n][k]

    constexpr int GROUP_M = 4;
    const int pid = blockIdx.x;
    const int T_m = a.gt.total_mtiles, T_n = a.ntiles;
    const int per_group = GROUP_M * T_n;
    const int first_m = (pid / per_group) * GROUP_M;
    const int gsz = (T_m - first_m) < GROUP_M ? (T_m - first_m) : GROUP_M;
    const int mt = first_m + (pid % per_group) % gsz;
    const int nt = (pid % per_group) / gsz;

    const int g = group_of_tile(a.gt, mt);
    const int rs = g ? a.gt.row_end[g - 1] : 0;
    const int r1 = a.gt.row_end[g];
    const int m0 = rs + (mt - a.gt.tile_start[g]) * GF_BM;
    const int vrows = r1 - m0;
    const int n0 = nt * GF_BN;
    const int64_t K = a.K, N = a.N;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    // Operand streams through buffer resources (offsets outside a resource read zeros).
    // A: rows [m0, r1) of x; thread chunks c = tid + 256 i: row c / KCH, k chunk c % KCH (8 elements).
    const __amdgpu_buffer_rsrc_t ares = make_rsrc((const uint16_t*)a.x + (int64_t)m0 * K,
                                                     (uint32_t)((vrows < GF_BM ? vrows : GF_BM) * K * 2));
    const __amdgpu_buffer_rsrc_t bres = make_rsrc((const uint16_t*)a.w + (int64_t)g * K * N, (uint32_t)(K * N * 2));
    uint32_t aoff[GF_CA], boff[GF_CB];
    int arow[GF_CA], akc[GF_CA], brow[GF_CB], bkc[GF_CB];
#pragma unroll
    for (int i = 0; i < GF_CA; ++i) {
        const int c = tid + NT * i;
        arow[i] = c / GF_KCH;
        akc[i] = c % GF_KCH;
        aoff[i] = arow[i] < vrows ? (uint32_t)((arow[i] * K + akc[i] * 8) * 2) : 0x80000000u;
    }
#pragma unroll
    for (int i = 0; i < GF_CB; ++i) {
        // weight [N][K]: like A, rows are output columns
        const int c = tid + NT * i;
        brow[i] = c / GF_KCH;
        bkc[i] = c % GF_KCH;
        const int n = n0 + brow[i];
        boff[i] = n < N ? (uint32_t)((n * K + bkc[i] * 8) * 2) : 0x80000000u;
    }
    // weight [K][N]: pair p = tid + NT i takes k rows 2 (p / NCH) and + 1 of n chunk p % NCH
    int bkp[GF_CP], bnc[GF_CP];
    bool bn_ok[GF_CP];
#pragma unroll
    for (int i = 0; i < GF_CP; ++i) {
        const int p2 = tid + NT * i;
        bkp[i] = p2 / NCH;
        bnc[i] = p2 % NCH;
        bn_ok[i] = n0 + bnc[i] * 8 < N;
    }
    const int nk = (int)((K + GF_BK - 1) / GF_BK);

    uint4 ra[GF_CA], rb[TRANS ? GF_CB : 2 * GF_CP];
    auto ld16 = [](__amdgpu_buffer_rsrc_t r, uint32_t off) {
        const v4i v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        return make_uint4((u32)v[0], (u32)v[1], (u32)v[2], (u32)v[3]);
    };
    auto load_stage = [&](int kt) {
        const int k0 = kt * GF_BK;
#pragma unroll
        for (int i = 0; i < GF_CA; ++i)
            ra[i] = ld16(ares, k0 + akc[i] * 8 < K ? aoff[i] + (uint32_t)(k0 * 2) : 0x80000000u);
        if constexpr (TRANS) {
#pragma unroll
            for (int i = 0; i < GF_CB; ++i)
                rb[i] = ld16(bres, k0 + bkc[i] * 8 < K ? boff[i] + (uint32_t)(k0 * 2) : 0x80000000u);
        } else {
#pragma unroll
            for (int i = 0; i < GF_CP; ++i)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int k = k0 + 2 * bkp[i] + h;
                    rb[2 * i + h] = ld16(bres, k < K && bn_ok[i] ? (uint32_t)((k * N + n0 + bnc[i] * 8) * 2) : 0x80000000u);
                }
        }
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < GF_CA; ++i)
            *reinterpret_cast<uint4*>(&As[buf][arow[i] * GF_PITCH + akc[i] * 8]) = ra[i];
        if constexpr (TRANS) {
#pragma unroll
            for (int i = 0; i < GF_CB; ++i)
                *reinterpret_cast<uint4*>(&Bs[buf][brow[i] * GF_PITCH + bkc[i] * 8]) = rb[i];
        } else {
            // 8 columns x 2 consecutive k: one 32-bit (k, k + 1) pair per column
#pragma unroll
            for (int i = 0; i < GF_CP; ++i)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const u32 lo = comp(rb[2 * i], j >> 1), hi = comp(rb[2 * i + 1], j >> 1);
                    const u32 pair = (j & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
                    *reinterpret_cast<u32*>(&Bs[buf][(bnc[i] * 8 + j) * GF_PITCH + 2 * bkp[i]]) = pair;
                }
        }
    };

    f32x16 acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;

    load_stage(0);
    store_stage(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_stage(kt + 1);  // in flight during this stage's MFMAs
#pragma unroll
        for (int kk = 0; kk < GF_BK / 16; ++kk) {
            // 32x32x16 operands: lane l holds row / column l % 32, k 8 (l / 32) .. + 7
            uint4 af[FM], bf[FN];
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
                af[fm] = *reinterpret_cast<const uint4*>(
                    &As[buf][(wm * TM + fm * 32 + (lane & 31)) * GF_PITCH + kk * 16 + (lane >> 5) * 8]);
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
                bf[fn] = *reinterpret_cast<const uint4*>(
                    &Bs[buf][(wn * TN + fn * 32 + (lane & 31)) * GF_PITCH + kk * 16 + (lane >> 5) * 8]);
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) {
                    if constexpr (BF16)
                        acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, af[fm]), __builtin_bit_cast(bf16x8, bf[fn]), acc[fm][fn], 0, 0, 0);
                    else
                        acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(f16x8, af[fm]), __builtin_bit_cast(f16x8, bf[fn]), acc[fm][fn], 0, 0, 0);
                }
        }
        if (kt + 1 < nk) store_stage(buf ^ 1);  // the other buffer was last read one stage ago
        __syncthreads();
    }

    // Epilogue.  32x32 C layout: lane l holds column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4.
    uint16_t* y = (uint16_t*)a.y;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
        const int64_t col = n0 + wn * TN + fn * 32 + (lane & 31);
        if (col >= N) continue;
        const float bv = a.bias_dt ? gf_load(a.bias, a.bias_dt, (int64_t)g * N + col) : 0.0f;
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int lrow = wm * TM + fm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (lrow < vrows) {
                    const float v = acc[fm][fn][r] + bv;
                    y[(int64_t)(m0 + lrow) * N + col] = BF16 ? f32_to_bf16_hw(v) : f32_to_f16(v);
                }
            }
    }
}

// 256 x 256 tiles on the int8 LDS core's structure: 8 waves (4 x 2) of 64 x 128, 64-deep stages
// (128 bytes of every operand row) DMA'd from global memory straight into a 2-stage LDS ring
// (buffer_load ... lds), one stage in flight while the other is multiplied.
//   x rows and a [N][K] weight: K-contiguous rows of 128 bytes, 16-byte chunks XOR-swizzled by
//   (row >> 1) & 7 (as the int8 core's A), fragments read with ds_read_b128.
//   a [K][N] weight: 64 rows of 256 columns (512 bytes), 16-byte chunks XOR-swizzled by 2 (k % 4);
//   fragments read with ds_read_b64_tr_b16: in each 16-lane group, lane s addresses row
//   k0 + s / 4, columns nb + 4 (s % 4) .. + 3, and lane j receives k0 .. k0 + 3 of column nb + j.
// Chunks past K or N point outside their buffer resource and read zeros.
constexpr int GL_BM = 256, GL_BN = 256, GL_BK = 64, GL_WN = 2, GL_NT = 512;  // 4 x 2 waves
constexpr int GL_ROWB = GL_BK * 2;                 // bytes per K-contiguous row and stage
constexpr int GL_A_BYTES = GL_BM * GL_ROWB;        // 32 KB
constexpr int GL_B_BYTES = GL_BN * GL_ROWB;        // 32 KB either layout
constexpr int GL_STAGE = GL_A_BYTES + GL_B_BYTES;
constexpr int GL_ISSUE = (GL_A_BYTES + GL_B_BYTES) / 16 / GL_NT;  // DMAs per thread per stage (8)

__device__ __forceinline__ int gl_swz(int r) { return (r >> 1) & 7; }

template <bool BF16, bool TRANS>
__global__ __launch_bounds__(GL_NT, 1) void gmm_lds_kernel(const GmmFArgs a)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    constexpr int GROUP_M = 4;
    const int pid = blockIdx.x;
    const int T_m = a.gt.total_mtiles, T_n = a.ntiles;
    const int per_group = GROUP_M * T_n;
    const int first_m = (pid / per_group) * GROUP_M;
    const int gsz = (T_m - first_m) < GROUP_M ? (T_m - first_m) : GROUP_M;
    const int mt = first_m + (pid % per_group) % gsz;
    const int nt = (pid % per_group) / gsz;
    const int g = group_of_tile(a.gt, mt);
    const int rs = g ? a.gt.row_end[g - 1] : 0;
    const int r1 = a.gt.row_end[g];
    const int m0 = rs + (mt - a.gt.tile_start[g]) * GL_BM;
    const int vrows = r1 - m0;
    const int n0 = nt * GL_BN;
    const int64_t K = a.K, N = a.N;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / GL_WN, wn = wave % GL_WN;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(CB_LDS uint8_t*)smem;

    const __amdgpu_buffer_rsrc_t ares = make_rsrc((const uint16_t*)a.x + (int64_t)m0 * K,
                                                     (uint32_t)((vrows < GL_BM ? vrows : GL_BM) * K * 2));
    const __amdgpu_buffer_rsrc_t bres = make_rsrc((const uint16_t*)a.w + (int64_t)g * K * N, (uint32_t)(K * N * 2));
    // per DMA i: the element offset of the chunk at k = 0 (or -1: nothing to fetch) and its k start
    int64_t aoff[4], boff[4];
    int akq[4], bk[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int cid = (i * 8 + wave) * 64 + lane;  // lane-linear 16-byte chunk of the stage
        const int row = cid >> 3, pos = cid & 7;
        const int q = pos ^ gl_swz(row);
        akq[i] = q * 8;
        aoff[i] = row < vrows ? (int64_t)row * K + q * 8 : -1;
        if constexpr (TRANS) {
            bk[i] = q * 8;
            boff[i] = n0 + row < N ? (int64_t)(n0 + row) * K + q * 8 : -1;
        } else {
            const int krow = cid >> 5, cpos = cid & 31;
            const int c = cpos ^ (2 * (krow & 3));  // logical 8-column chunk
            bk[i] = krow;
            boff[i] = n0 + c * 8 < N ? (int64_t)krow * N + n0 + c * 8 : -1;
        }
    }
    const int nk = (int)((K + GL_BK - 1) / GL_BK);
    auto issue = [&](int kt) {
        const uint32_t sa = lds_base + (uint32_t)((kt & 1) * GL_STAGE);
        const int k0 = kt * GL_BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const bool ok = aoff[i] >= 0 && k0 + akq[i] < K;
            dma16(ares, ok ? (uint32_t)((aoff[i] + k0) * 2) : 0x80000000u,
                  __builtin_amdgcn_readfirstlane(sa + (uint32_t)((i * 8 + wave) * 1024)));
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            bool ok;
            int64_t off;
            if constexpr (TRANS) {
                ok = boff[i] >= 0 && k0 + bk[i] < K;
                off = boff[i] + k0;
            } else {
                ok = boff[i] >= 0 && k0 + bk[i] < K;
                off = boff[i] + (int64_t)k0 * N;
            }
            dma16(bres, ok ? (uint32_t)(off * 2) : 0x80000000u,
                  __builtin_amdgcn_readfirstlane(sa + GL_A_BYTES + (uint32_t)((i * 8 + wave) * 1024)));
        }
    };

    f32x16 acc[2][4];
#pragma unroll
    for (int fm = 0; fm < 2; ++fm)
#pragma unroll
        for (int fn = 0; fn < 4; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0.0f;

    issue(0);
    issue(1);
    for (int kt = 0; kt < nk; ++kt) {
        wait_vmcnt_barrier<GL_ISSUE>();  // stage kt has landed (stage kt + 1 may stay in flight)
        const CB_LDS uint8_t* st = (const CB_LDS uint8_t*)smem + (kt & 1) * GL_STAGE;
#pragma unroll
        for (int ks = 0; ks < GL_BK / 16; ++ks) {
            uint4 af[2], bfr[4];
            const int q = 2 * ks + (lane >> 5);
#pragma unroll
            for (int fm = 0; fm < 2; ++fm) {
                const int r = wm * 64 + fm * 32 + (lane & 31);
                af[fm] = __builtin_bit_cast(uint4, *(const CB_LDS v4i*)(st + r * GL_ROWB + ((q ^ gl_swz(r)) << 4)));
            }
#pragma unroll
            for (int fn = 0; fn < 4; ++fn) {
                if constexpr (TRANS) {
                    const int r = wn * 128 + fn * 32 + (lane & 31);
                    bfr[fn] = __builtin_bit_cast(uint4, *(const CB_LDS v4i*)(st + GL_A_BYTES + r * GL_ROWB + ((q ^ gl_swz(r)) << 4)));
                } else {
                    const int grp = lane >> 4, s = lane & 15;
                    const int nb = wn * 128 + fn * 32 + 16 * (grp & 1);
                    const int col = nb + 4 * (s & 3);
                    u32 w[4];
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const int k = ks * 16 + 8 * (grp >> 1) + 4 * h + (s >> 2);
                        const int chunk = (col >> 3) ^ (2 * (k & 3));
                        const v4i16 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                            (CB_LDS v4i16*)(st + GL_A_BYTES + k * (GL_BN * 2) + chunk * 16 + (col & 7) * 2));
                        w[2 * h] = (u32)(uint16_t)v[0] | ((u32)(uint16_t)v[1] << 16);
                        w[2 * h + 1] = (u32)(uint16_t)v[2] | ((u32)(uint16_t)v[3] << 16);
                    }
                    bfr[fn] = make_uint4(w[0], w[1], w[2], w[3]);
                }
            }
#pragma unroll
            for (int fm = 0; fm < 2; ++fm)
#pragma unroll
                for (int fn = 0; fn < 4; ++fn) {
                    if constexpr (BF16)
                        acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                            __builtin_bit_cast(bf16x8, af[fm]), __builtin_bit_cast(bf16x8, bfr[fn]), acc[fm][fn], 0, 0, 0);
                    else
                        acc[fm][fn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                            __builtin_bit_cast(f16x8, af[fm]), __builtin_bit_cast(f16x8, bfr[fn]), acc[fm][fn], 0, 0, 0);
                }
        }
        // every wave is done with this buffer before the DMA of stage kt + 2 overwrites it
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        issue(kt + 2);  // past K: fetches nothing
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // Epilogue.  32x32 C layout: lane l holds column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4.
    // Rows r and r + 1 of a lane pair (l, l ^ 1) are swapped so that each lane stores two adjacent
    // columns of one row as one dword: the even lane row r, columns (c, c + 1), the odd lane row
    // r + 1, columns (c - 1, c).  Rows past the group's end fall outside the resource and are dropped.
    const __amdgpu_buffer_rsrc_t ores = make_rsrc((uint16_t*)a.y + (int64_t)m0 * N,
                                                  (uint32_t)((vrows < GL_BM ? vrows : GL_BM) * N * 2));
    const bool odd = lane & 1;
    float bv[4];
    uint32_t coff[4];
#pragma unroll
    for (int fn = 0; fn < 4; ++fn) {
        const int64_t col = n0 + wn * 128 + fn * 32 + (lane & 31);
        bv[fn] = a.bias_dt ? gf_load(a.bias, a.bias_dt, (int64_t)g * N + (col < N ? col : 0)) : 0.0f;
        coff[fn] = col < N ? (uint32_t)(col & ~(int64_t)1) * 2u : 0x80000000u;
    }
#pragma unroll
    for (int fm = 0; fm < 2; ++fm)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            const int lrow = wm * 64 + fm * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);  // rows lrow, lrow + 1
            const uint32_t roff = (uint32_t)(lrow + (odd ? 1 : 0)) * (uint32_t)N * 2u;
#pragma unroll
            for (int fn = 0; fn < 4; ++fn) {
                const float v0 = acc[fm][fn][r] + bv[fn], v1 = acc[fm][fn][r + 1] + bv[fn];
                const uint32_t h0 = BF16 ? f32_to_bf16_hw(v0) : f32_to_f16(v0);
                const uint32_t h1 = BF16 ? f32_to_bf16_hw(v1) : f32_to_f16(v1);
                const uint32_t p = h0 | (h1 << 16);
                // partner lane's pair (quad_perm [1, 0, 3, 2])
                const uint32_t q = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)p, 0xB1, 0xF, 0xF, false);
                const uint32_t w = odd ? ((q >> 16) | (p & 0xffff0000u)) : ((p & 0xffffu) | (q << 16));
                __builtin_amdgcn_raw_buffer_store_b32(w, ores, roff + coff[fn], 0, 0);
            }
        }
}

// Any dtype and layout: one output element per thread iteration (grid-stride), fp32 accumulation
// in k order, the bias added in fp32, one narrowing to the output dtype.
__global__ __launch_bounds__(256) void gmm_generic_kernel(const GmmFArgs a)
{
    const int64_t total = a.M * a.N;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int row = (int)(i / a.N);
        const int64_t col = i % a.N;
        const int g = group_of_row(a.gt, row);
        const int64_t wb = (int64_t)g * a.K * a.N;
        float acc = 0.0f;
        for (int64_t k = 0; k < a.K; ++k) {
            const float xv = gf_load(a.x, a.x_dt, (int64_t)row * a.K + k);
            const float wv = gf_load(a.w, a.x_dt, wb + (a.trans ? col * a.K + k : k * a.N + col));
            acc = acc + xv * wv;
        }
        if (a.bias_dt) acc = acc + gf_load(a.bias, a.bias_dt, (int64_t)g * a.N + col);
        gf_store(a.y, a.x_dt, i, acc);
    }
}

// A test override of 128 selects the 128 x 128 register-staged kernel for every fp16/bf16 shape (it
// is otherwise taken only where a 256-row block of x or y passes 2 GiB).
static bool gmm_lds_enabled() { return g_overrides.gmm_tile != 128; }

// Raise a kernel's dynamic LDS limit once per (kernel, device).
static void set_dynamic_lds_once(const void* kern, int bytes)
{
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    int dev = -1;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(mu);
    if (done.insert({kern, dev}).second)
        (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

}  // namespace cb

using namespace cb;

// The reference's launch_gmm (grouped_matmul_launch.h:66-70) with the plugin's checks
// (grouped_matmul_plugin.cpp:127-157, in order) moved behind a status return.  K = 0 writes the
// bias (or zeros).
extern "C" int cb_grouped_matmul(const void* x, const void* weight, const void* bias, int x_dtype, int bias_dtype,
                                 const int64_t* group_list, int64_t group_len, int64_t M, int64_t K, int64_t N,
                                 int64_t E, int transpose_weight, void* y, void* stream)
{
    if (M < 0 || K < 0 || N < 0 || E < 0) return CB_ERR_SHAPE;
    if (E < 1 || E > kGmmMaxExperts) return CB_ERR_GROUP_COUNT;  // plugin :138-139
    if (x_dtype != CB_DT_FLOAT16 && x_dtype != CB_DT_BFLOAT16 && x_dtype != CB_DT_FLOAT32) return CB_ERR_DTYPE;
    if (bias && bias_dtype != CB_DT_FLOAT16 && bias_dtype != CB_DT_BFLOAT16 && bias_dtype != CB_DT_FLOAT32)
        return CB_ERR_DTYPE;
    const int vs = validate_group_list(group_list, group_len, E, M);
    if (vs != CB_OK) return vs;
    if (M == 0 || N == 0) return CB_OK;
    if (!x && K > 0) return CB_ERR_NULL_POINTER;
    if ((!weight && K > 0) || !y) return CB_ERR_NULL_POINTER;
    if (M > 0x7fffffffLL) return CB_ERR_SHAPE;

    GmmFArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = x;
    a.w = weight;
    a.bias = bias;
    a.y = y;
    a.M = M;
    a.K = K;
    a.N = N;
    a.x_dt = x_dtype;
    a.bias_dt = bias ? bias_dtype : 0;
    a.trans = transpose_weight ? 1 : 0;
    hipStream_t st = (hipStream_t)stream;
    TimedLaunch timed(st);

    const bool mfma = x_dtype != CB_DT_FLOAT32 && K > 0 && K % 8 == 0 && N % 8 == 0 && aligned(x, 16) &&
                      aligned(weight, 16) && K * N * 2 < (1LL << 31) && 128 * K * 2 < (1LL << 31);
    if (mfma) {
        if (gmm_lds_enabled() && 256 * K * 2 < (1LL << 31) && 256 * N * 2 < (1LL << 31)) {
            build_group_table(a.gt, group_list, E, GL_BM);
            a.ntiles = (int)((N + GL_BN - 1) / GL_BN);
            const int64_t blocks = (int64_t)a.gt.total_mtiles * a.ntiles;
            if (blocks <= 0) return CB_OK;
            const bool bf = x_dtype == CB_DT_BFLOAT16;
            const void* kern = bf ? (a.trans ? (const void*)gmm_lds_kernel<true, true> : (const void*)gmm_lds_kernel<true, false>)
                                  : (a.trans ? (const void*)gmm_lds_kernel<false, true> : (const void*)gmm_lds_kernel<false, false>);
            set_dynamic_lds_once(kern, 2 * GL_STAGE);
            if (bf && a.trans) hipLaunchKernelGGL((gmm_lds_kernel<true, true>), dim3((unsigned)blocks), dim3(GL_NT), 2 * GL_STAGE, st, a);
            else if (bf) hipLaunchKernelGGL((gmm_lds_kernel<true, false>), dim3((unsigned)blocks), dim3(GL_NT), 2 * GL_STAGE, st, a);
            else if (a.trans) hipLaunchKernelGGL((gmm_lds_kernel<false, true>), dim3((unsigned)blocks), dim3(GL_NT), 2 * GL_STAGE, st, a);
            else hipLaunchKernelGGL((gmm_lds_kernel<false, false>), dim3((unsigned)blocks), dim3(GL_NT), 2 * GL_STAGE, st, a);
            return check_launch();
        }
        build_group_table(a.gt, group_list, E, 128);
        a.ntiles = (int)((N + 127) / 128);
        const int64_t blocks = (int64_t)a.gt.total_mtiles * a.ntiles;
        if (blocks <= 0) return CB_OK;
        const dim3 grid((unsigned)blocks);
        const bool bf = x_dtype == CB_DT_BFLOAT16;
        if (bf && a.trans) hipLaunchKernelGGL((gmm_mfma_kernel<true, true, 128, 128, 2, 2>), grid, dim3(256), 0, st, a);
        else if (bf) hipLaunchKernelGGL((gmm_mfma_kernel<true, false, 128, 128, 2, 2>), grid, dim3(256), 0, st, a);
        else if (a.trans) hipLaunchKernelGGL((gmm_mfma_kernel<false, true, 128, 128, 2, 2>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((gmm_mfma_kernel<false, false, 128, 128, 2, 2>), grid, dim3(256), 0, st, a);
        return check_launch();
    }
    build_group_table(a.gt, group_list, E, 1);
    const int64_t total = M * N;
    const int64_t blocks = (total + 255) / 256;
    hipLaunchKernelGGL(gmm_generic_kernel, dim3((unsigned)(blocks < 65536 ? blocks : 65536)), dim3(256), 0, st, a);
    return check_launch();
}
