// gemm_pf.hpp - persistent int8 GEMM with the dequant epilogue (QuantMatmul, the grouped
// down-projection GroupedMatmulQuant) on the GroupedMatmulSwigluQuant prefill core.
//
// Reference being replaced: the cube GEMM + vector dequant of quant_matmul (quant_matmul_plugin.cpp
// launch path) and of the grouped int8 matmul; here the int32 product never leaves the registers.
//
// Core (gmsq_prefill.hpp): 256 x 256 tiles, four waves of 128 x 128 (v_mfma_i32_32x32x32_i8), K in
// 64-deep stages through a 4-slot LDS ring fed by buffer_load ... lds, the DMAs of a stage spread
// over the MFMAs of the previous one, and one continuous stage stream per workgroup: the last
// iterations of a tile fetch the next tile's first 3.5 stages.  The column tile is folded into the
// weight resource (its base is the tile's first column), so the per-lane chunk offsets are the
// same for every tile of the launch.
//
// Epilogue, register direct (the ring already receives the next tile's stages): the dequant chain
// of apply_deq per element (the common chain - per-channel scale, optional per-token scale, bf16
// out - without the selects), a 4 x 4 transpose of 16-bit values across each lane quad so that a
// lane holds 4 consecutive columns of one row, and stores through a resource over the
// tile's valid rows (columns past N go outside it), after a swap between lanes c and c ^ 4 that
// gives each lane 8 columns of one row, so the stores are 16 bytes.
#pragma once

#include "gmsq_prefill.hpp"

namespace cb {

constexpr int kGpfLds = kPfRing + 2 * kPfScSlot;  // the ring, then two scale slots

// The tile's plan: rows [m0, m0 + vrows) of group g, column tile nt.
struct GpfTile {
    int g, m0, vrows, nt;
};

// Launch order (two maps; the block map below where it applies, measured 2-4% faster on grouped
// prefill-shaped GEMMs with 16 column tiles and level on QuantMatmul).
// Run map.  Tiles k are numbered row-group major: groups of G consecutive row tiles, within a
// group column tile by column tile, row tile fastest - G consecutive tiles share a weight slab.
// Slot p (workgroup blockIdx.x walks p = blockIdx.x, + gridDim.x, ...; it runs on XCD p % 8 when
// gridDim.x is a multiple of 8) takes tile k = G (8 (q / G) + p % 8) + q % G with q = p / 8: each
// run of G tiles sharing a weight slab goes to one XCD, whose workgroups run it together, so the
// slab crosses into one L2 once.  Slots past the padded count or with k >= T take no tile.
// (G = 1, 4, 8, 16 measured within noise of each other.)
constexpr int kGpfG = 8;

// Block map (T_n a multiple of 8, at least 4 row tiles): the tiles form blocks of 4 row tiles x 8
// column tiles (tile i of a block: row tile i % 4, column tile i / 4), blocks numbered row band
// major; slot p = 8 q + x takes tile q % 32 of block 8 (q / 32) + x, so in each round of 256 slots
// every XCD runs one whole block: 4 activation slabs and 8 weight slabs per stage in its L2 (the
// run map gives an XCD 16 and 2 at 16 column tiles).  Tiles past the last row tile take no slot.
__host__ __device__ inline bool gpf_block_map(const int T_m, const int T_n)
{
    return T_n % 8 == 0 && T_m >= 4;
}

struct GpfMap {
    bool block;
    int T_m, T_n, slots, total;
};

__device__ __forceinline__ GpfMap gpf_map(const GemmArgs& a)
{
    GpfMap m;
    m.T_m = a.gt.total_mtiles;
    m.T_n = a.ntiles;
    m.block = gpf_block_map(m.T_m, m.T_n);
    if (m.block) {
        const int nblk = (m.T_m + 3) / 4 * (m.T_n / 8);
        m.total = nblk * 32;
        m.slots = (nblk + 7) / 8 * 256;
    } else {
        m.total = m.T_m * m.T_n;
        m.slots = (m.total + 8 * kGpfG - 1) / (8 * kGpfG) * (8 * kGpfG);
    }
    return m;
}

// Slot p -> tile number k, or -1 when the slot takes no tile.
__device__ __forceinline__ int gpf_k_of_slot(const GpfMap& m, const int p)
{
    const int x = p & 7, q = p >> 3;
    if (m.block) {
        const int k = (8 * (q >> 5) + x) * 32 + (q & 31);
        return (k < m.total && ((k >> 5) / (m.T_n >> 3)) * 4 + (k & 3) < m.T_m) ? k : -1;
    }
    const int k = kGpfG * (8 * (q / kGpfG) + x) + q % kGpfG;
    return k < m.total ? k : -1;
}

__device__ __forceinline__ GpfTile gpf_tile(const GemmArgs& a, const GpfMap& m, const int k)
{
    int mt;
    GpfTile t;
    if (m.block) {
        const int nb = m.T_n >> 3, blk = k >> 5, i = k & 31;
        mt = (blk / nb) * 4 + (i & 3);
        t.nt = (blk % nb) * 8 + (i >> 2);
    } else {
        const int per_group = kGpfG * m.T_n;
        const int first_m = (k / per_group) * kGpfG;
        const int gsz = (m.T_m - first_m) < kGpfG ? (m.T_m - first_m) : kGpfG;
        mt = first_m + (k % per_group) % gsz;
        t.nt = (k % per_group) / gsz;
    }
    t.g = group_of_tile(a.gt, mt);
    t.m0 = (t.g ? a.gt.row_end[t.g - 1] : 0) + (mt - a.gt.tile_start[t.g]) * 256;
    t.vrows = a.gt.row_end[t.g] - t.m0;
    return t;
}

// The first slot p' >= p (in steps of the grid) that takes a tile, or -1.
__device__ __forceinline__ int gpf_next_slot(const GpfMap& m, int p, const int step)
{
    for (; p < m.slots; p += step)
        if (gpf_k_of_slot(m, p) >= 0) return p;
    return -1;
}

__device__ __forceinline__ PfSrc gpf_src(const GemmArgs& a, const GpfTile& t)
{
    PfSrc s;
    const int64_t K = a.K, N = a.N;
    const int64_t c0 = (int64_t)t.nt * 256;
    s.ares = make_rsrc(a.x + (int64_t)t.m0 * K, (uint32_t)((int64_t)(t.vrows < 256 ? t.vrows : 256) * K));
    s.bres = make_rsrc(a.w + (int64_t)t.g * a.w_gstride + c0, (uint32_t)(K * N - c0));
#pragma unroll
    for (int i = 0; i < 4; ++i) s.ga[i] = 0x80000000u;
    return s;
}

// Row scale (the per-token scale, 1 without one) of tile row tid and column scale of tile column
// tid, loaded into registers (every thread loads, absent operands through empty resources).
__device__ __forceinline__ PfScales gpf_scales(const GemmArgs& a, const GpfTile& t)
{
    const EpiArgs& e = a.epi;
    const int tid = opaque((int)threadIdx.x);
    PfScales s;
    const __amdgpu_buffer_rsrc_t pres =
        e.has_pt ? make_rsrc(e.pertoken + t.m0, (uint32_t)((t.vrows < 256 ? t.vrows : 256) * 4)) : make_rsrc(a.x, 0u);
    const float v = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(pres, (uint32_t)((tid < t.vrows ? tid : t.vrows - 1) * 4), 0, 0));
    s.xs = e.has_pt ? v : 1.0f;
    const int64_t cc = (int64_t)t.nt * 256 + tid;
    const int64_t si = (int64_t)t.g * e.scale_gstride + (e.scale_perchan ? (cc < a.N ? cc : 0) : 0);
    const __amdgpu_buffer_rsrc_t s32 = make_rsrc(e.scale, e.scale_bf16 ? 0u : 0x80000000u);
    const __amdgpu_buffer_rsrc_t s16 = make_rsrc(e.scale, e.scale_bf16 ? 0x80000000u : 0u);
    const float f32 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s32, (uint32_t)(si * 4), 0, 0));
    const uint16_t b16 = __builtin_amdgcn_raw_buffer_load_b16(s16, (uint32_t)(si * 2), 0, 0);
    s.cs = e.scale_bf16 ? bf16_to_f32(b16) : f32;
    return s;
}

// 16-bit 4 x 4 transpose across the lane quad (qi = lane % 4): on entry the lane holds rows
// 0..3 of its column as p01 = rows 0, 1 and p23 = rows 2, 3; on exit d0, d1 hold row qi, columns
// 0..3 of the quad.  Step 1 trades 2-row halves with lane qi ^ 2, step 2 single values with qi ^ 1;
// the lane-dependent choices are selects and per-lane byte selectors of v_perm_b32 (sel_*), not
// branches.
struct Quad16Sel {
    bool hi2;
    u32 s_send, s_d0, s_d1;
};

__device__ __forceinline__ Quad16Sel quad16_sel(const int qi)
{
    const bool odd = qi & 1;
    Quad16Sel q;
    q.hi2 = qi & 2;
    q.s_send = odd ? 0x05040100u : 0x07060302u;  // perm(second, first): lo / hi halves of both
    q.s_d0 = odd ? 0x03020504u : 0x05040100u;    // perm(r2, first)
    q.s_d1 = odd ? 0x03020706u : 0x07060100u;    // perm(r2, second)
    return q;
}

__device__ __forceinline__ void quad_transpose16(const u32 p01, const u32 p23, const Quad16Sel& q, u32& d0, u32& d1)
{
    const u32 recv = (u32)__builtin_amdgcn_mov_dpp((int)(q.hi2 ? p01 : p23), 0x4E, 0xF, 0xF, false);
    // first: column qi & 1, second: column (qi & 1) + 2, both for the lane pair's two rows
    const u32 first = q.hi2 ? recv : p01, second = q.hi2 ? p23 : recv;
    const u32 r2 = (u32)__builtin_amdgcn_mov_dpp((int)__builtin_amdgcn_perm(second, first, q.s_send), 0xB1, 0xF,
                                                     0xF, false);
    d0 = __builtin_amdgcn_perm(r2, first, q.s_d0);
    d1 = __builtin_amdgcn_perm(r2, second, q.s_d1);
}

// Two values rounded to bf16 (round to nearest even) in one dword, the first in the low half.
__device__ __forceinline__ u32 pack_bf16x2(const float a, const float b)
{
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(u32, __builtin_convertvector(f32x2{a, b}, bf16x2));
}

// The dequant epilogue of one tile from the accumulators.  Lane (h = lane / 32, c = lane % 32) of
// fragment (fm, fn) holds rows (2 fm + wm) * 32 + 8 (r / 4) + 4 h + r % 4, column
// tcol(fn) + c with tcol(fn) = 128 (fn / 2) + 64 wn + 32 (fn % 2).
template <bool SIMPLE>
__device__ __forceinline__ void gpf_epilogue(const GemmArgs& a, uint8_t* smem, v16i (&acc)[4][4], const GpfTile& t,
                                             const int par)
{
    const int tid = opaque((int)threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const EpiArgs& e = a.epi;
    const int64_t N = a.N;
    const int h = lane >> 5, c = lane & 31, qi = c & 3;
    const Quad16Sel qs = quad16_sel(qi);
    const CB_LDS float* xs_l = (const CB_LDS float*)((CB_LDS uint8_t*)smem + kPfSc + par * kPfScSlot);
    const CB_LDS float* cs_l = xs_l + 256;
    const int vr = t.vrows < 256 ? t.vrows : 256;
    const __amdgpu_buffer_rsrc_t ores = make_rsrc((uint16_t*)e.out + (int64_t)t.m0 * N, (uint32_t)((int64_t)vr * N * 2));
    ColDeq cd[4];
#pragma unroll
    for (int fn = 0; fn < 4; ++fn) {
        const int tc = (fn >> 1) * 128 + wn * 64 + (fn & 1) * 32;
        const int64_t cc = (int64_t)t.nt * 256 + tc + c;  // this lane's column (values)
        if constexpr (SIMPLE) cd[fn] = ColDeq{cs_l[tc + c], 0.0f, 0.0f};
        else cd[fn] = col_deq(e, t.g, 0, cc < N ? cc : 0);
    }
    // the dequant chain of lane value i of accumulator slice (fm, fn, q) -> bf16 / fp16 pairs
    auto packed = [&](const int fm, const int fn, const int q, const v4f& xs4, u32& p01, u32& p23) {
        float f[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int acc_v = acc_read(acc[fm][fn][4 * q + i]);
            if constexpr (SIMPLE) f[i] = ((float)acc_v * cd[fn].scale) * xs4[i];
            else f[i] = apply_deq(e, cd[fn], acc_v, xs4[i]);
        }
        if (SIMPLE || e.out_bf16) {
            p01 = pack_bf16x2(f[0], f[1]);
            p23 = pack_bf16x2(f[2], f[3]);
        } else {
            p01 = (u32)f32_to_f16(f[0]) | ((u32)f32_to_f16(f[1]) << 16);
            p23 = (u32)f32_to_f16(f[2]) | ((u32)f32_to_f16(f[3]) << 16);
        }
    };
    // 16-byte stores (the launch requires N % 8 == 0 and a 16-byte aligned output).
    // 16-byte stores: after the quad transposes of slices q and q + 1, lanes c and c ^ 4 hold
    // columns 0..3 and 4..7 of the same 8-column group for rows of both slices; the lane with
    // bit 2 of c clear keeps slice q's row and takes columns 4..7 from lane c + 4, the other
    // keeps slice q + 1's row and takes columns 0..3 from lane c - 4, so each lane stores 8
    // contiguous columns of one row
    const bool hi4 = (c >> 2) & 1;
    uint32_t coff8[4];
#pragma unroll
    for (int fn = 0; fn < 4; ++fn) {
        const int64_t c8 = (int64_t)t.nt * 256 + (fn >> 1) * 128 + wn * 64 + (fn & 1) * 32 + (c & ~7);
        coff8[fn] = c8 < N ? (uint32_t)c8 * 2u : 0x80000000u;
    }
#pragma unroll
    for (int fm = 0; fm < 4; ++fm) {
#pragma unroll
        for (int qp = 0; qp < 2; ++qp) {
            const int row0 = (2 * fm + wm) * 32 + 16 * qp + 4 * h;  // slice 2 qp; slice 2 qp + 1 is 8 rows on
            const v4f xa = *(const CB_LDS v4f*)(xs_l + row0);
            const v4f xb = *(const CB_LDS v4f*)(xs_l + row0 + 8);
            const uint32_t roff = (uint32_t)(row0 + (hi4 ? 8 : 0) + qi) * (uint32_t)N * 2u;
#pragma unroll
            for (int fn = 0; fn < 4; ++fn) {
                u32 pa01, pa23, pb01, pb23, x0, x1, z0, z1;
                packed(fm, fn, 2 * qp, xa, pa01, pa23);
                packed(fm, fn, 2 * qp + 1, xb, pb01, pb23);
                quad_transpose16(pa01, pa23, qs, x0, x1);
                quad_transpose16(pb01, pb23, qs, z0, z1);
                // one lane-uniform exchange with lane c ^ 4 (ds_swizzle bit mode, xor mask 4): a
                // cross-lane read under a lane-dependent branch would see inactive lanes
                const u32 s0 = hi4 ? x0 : z0, s1 = hi4 ? x1 : z1;
                const u32 r0 = (u32)__builtin_amdgcn_ds_swizzle((int)s0, 0x101F);
                const u32 r1 = (u32)__builtin_amdgcn_ds_swizzle((int)s1, 0x101F);
                typedef unsigned int v4u __attribute__((ext_vector_type(4)));
                const v4u w = hi4 ? v4u{r0, r1, z0, z1} : v4u{x0, x1, r0, r1};
                __builtin_amdgcn_raw_buffer_store_b128(w, ores, roff + coff8[fn], 0, 0);
            }
        }
    }
}

// Persistent launch: gridDim.x workgroups (at most one per CU) walk the launch order's slots.
// Batch 1, K of at least 4 stages, N a multiple of 8 and the output 16-byte aligned (16-byte
// stores), bf16 / fp16 out.
template <bool SIMPLE>
__global__ __launch_bounds__(256, 1) void gpf_dequant_kernel(const GemmArgs a)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const GpfMap map = gpf_map(a);
    const int step = (int)gridDim.x;
    int pid = gpf_next_slot(map, (int)blockIdx.x, step);
    if (pid < 0) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    uint32_t a_rd[4][2], b_rd[4];
    pf_read_offsets(wm, wn, lane, a_rd, b_rd);
    const int nk = __builtin_amdgcn_readfirstlane((int)((a.K + PfCfg::BK - 1) / PfCfg::BK));
    const PfOffs offs = pf_offsets<false, false>(a, wave, lane);
    auto put_scales = [&](const PfScales& v, int par) {
        CB_LDS float* sl = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfSc + par * kPfScSlot);
        sl[tid] = v.xs;
        sl[256 + tid] = v.cs;
    };
    GpfTile cur_t = gpf_tile(a, map, gpf_k_of_slot(map, pid));
    PfSrc cur = gpf_src(a, cur_t);
    pf_prologue<false>(cur, offs, nk, smem, wave);
    put_scales(gpf_scales(a, cur_t), 0);
    int par = 0, rb = 0;
    bool first = true;
    for (;;) {
        const int pn = gpf_next_slot(map, pid + step, step);
        const bool has_nxt = pn >= 0;
        GpfTile nxt_t;
        PfSrc nxt;
        PfScales nsc;
        if (has_nxt) {
            nxt_t = gpf_tile(a, map, gpf_k_of_slot(map, pn));
            nxt = gpf_src(a, nxt_t);
            nsc = gpf_scales(a, nxt_t);
        } else {
            nxt = pf_dead(a);
        }
        v16i acc[4][4];  // defined by the K loop (its first MFMAs start from zero)
        const int nblk = (cur_t.vrows + 31) / 32;
        const int nv = __builtin_amdgcn_readfirstlane(nblk > wm ? min((nblk - wm + 1) / 2, 4) : 0);
        // A later tile's loop starts with wait vmcnt(63): its first 28 DMAs were issued before the
        // previous epilogue's 64 stores, so at most 63 outstanding operations means they landed.
        if (nv >= 4) pf_kloop<4, true, false>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
        else if (nv == 3) pf_kloop<3, true, false>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
        else if (nv == 2) pf_kloop<2, true, false>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
        else if (nv == 1) pf_kloop<1, true, false>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
        else pf_kloop<0, true, false>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
        gpf_epilogue<SIMPLE>(a, smem, acc, cur_t, par);
        if (has_nxt) put_scales(nsc, par ^ 1);
        // every wave is past this epilogue's scale reads (and the next scales are written) before
        // the next tile's epilogue; no global load in between, so no wait on the stores
        __syncthreads();
        if (!has_nxt) break;
        rb = (rb + nk) & 3;
        par ^= 1;
        cur = nxt;
        cur_t = nxt_t;
        pid = pn;
        first = false;
    }
}

}  // namespace cb
