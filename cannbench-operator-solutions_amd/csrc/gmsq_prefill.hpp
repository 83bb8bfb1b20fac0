// gmsq_prefill.hpp - GroupedMatmulSwigluQuant for prefill-shaped groups: the int8 grouped GEMM,
// the dequant + SwiGLU epilogue and the per-token int8 requant in one persistent launch.
//
// Reference being replaced: launch_gmsq_cube (gmsq_cube_kernel.cpp:48-130, 139-162) writes the
// int32 product [M, N] to a workspace and launch_gmsq_vec (gmsq_vec_kernel.cpp:58-270) reads it
// back for the dequant, SwiGLU and requant.  Here the int32 product and the fp32 activation stay in
// registers; the only cross-workgroup traffic is one row abs-max per (row, column tile).
//
// Tile: 256 rows x 256 weight columns (the 128 gate columns nt*128.. and the matching 128 up
// columns H + nt*128..), K in 64-deep stages through a 4-slot LDS ring (4 x 32 KB).  Four waves,
// one per SIMD, each own a 128 x 128 block (4 x 4 fragments of v_mfma_i32_32x32x32_i8, 256
// accumulator registers): per 32-deep step a wave reads 4 A and 4 B fragments (8 KB) for 16
// MFMAs, a third less LDS traffic per MFMA than 64 x 128 wave blocks.
//
// Stage stream.  A stage is 16 A and 16 B DMA chunks of 1 KB (buffer_load_dwordx4 ... lds); each
// wave issues 4 A and 4 B chunks per stage, spread one per 4 MFMAs instead of in a burst:
//   iteration kt, half 1 (MFMAs of step 0): the B chunks of stage kt + 3
//   barrier (stage kt + 1 has landed; every wave has finished reading stage kt)
//   iteration kt, half 2 (MFMAs of step 1): the A chunks of stage kt + 4 into stage kt's slot
// so 2.5 stages (80 KB) are in flight while one is multiplied.  The stream runs on across tiles:
// the stages past K are the workgroup's next tile's first 3.5 stages (its prologue), issued while
// the last stages of this tile are multiplied, so they arrive during this tile's epilogue and no
// tile starts with a burst of DMAs.  Stage kt of a tile lives in ring slot (rb + kt) % 4.
//
// Epilogue, per tile (it does not touch the ring; the tile's scales sit in one of two LDS slots,
// written during the previous tile's epilogue):
//   1. SwiGLU from the accumulators (the reference's operation order), |act| row maxima reduced
//      across lanes (DPP) and across the two waves sharing rows (LDS), one device-scope atomicMax
//      per (row, tile), one arrival on the row tile's counter;
//   2. the activations stay in VGPRs through the workgroup's next K loop; after it, the row tile's
//      counter is checked (its other 15 column tiles have normally arrived long before), and the
//      tile is requantised: per-row 127 / amax through LDS, rint16 in registers, a 4 x 4 byte
//      transpose across each lane quad, dword stores of int8 y (four consecutive columns per lane).
// The column tile of a workgroup rotates by one per round, so the two column tiles whose weight
// lines read slowly fall to a different workgroup every round.  A column tile whose wait times out
// marks itself in the workspace and stores nothing; the fix-up launch that always follows
// recomputes exactly those tiles with the final row maxima, so the output is right whatever the
// residency of the grid (it exits at once when nothing is marked).  K below 4 stages (no stage
// stream across tiles) uses the lock-step form: each tile waits for its row tile's exchange and
// requantises at once.
#pragma once

#include "gemm_lds.hpp"

namespace cb {


using PfCfg = LdsCfg<2, 2, 4, 64>;

// DMA plan.  A lane's chunk offsets within a stage depend only on the workgroup's column tile
// (fixed for the launch) and, for contiguous rows, not on the row tile at all: PfOffs holds them
// once per workgroup, and a tile contributes only its two buffer resources (PfSrc; rows past the
// tile's valid rows lie outside the activation resource and read zeros).  Gathered rows (GATHER)
// add per-tile source-row offsets.
// Chunk i of a wave's 4 A (B) chunks lies i * ka (16 weight rows) bytes past chunk 0, so a lane keeps
// one offset per operand and the rest is a scalar.
struct PfOffs {
    uint32_t a0, b0;
    uint32_t ka;  // 64 activation rows (0 with GATHER: the row offsets are per chunk)
    uint32_t n;   // weight row length
};
struct PfSrc {
    __amdgpu_buffer_rsrc_t ares, bres;
    uint32_t ga[4];  // GATHER: source row * K of each A chunk (0x80000000: no row)
};

// SW (GroupedMatmulSwigluQuant): the stage's 256 columns are a column tile's 128 gate columns then
// the matching 128 up columns, counted from the weight resource's base, which pf_src places at
// the tile's first gate column (so these offsets are the same for every column tile).  Otherwise
// 256 consecutive columns from the start of the weight resource, which the caller places at the
// tile's first column.
template <bool GATHER, bool SW = true>
__device__ __forceinline__ PfOffs pf_offsets(const GemmArgs& a, const int wave, const int lane)
{
    PfOffs o;
    const uint32_t K = (uint32_t)a.K;
    o.n = (uint32_t)a.N;
    o.ka = GATHER ? 0u : 64u * K;
    {
        // chunk 0: A tile row wave * 16 + lane / 4; the swizzle depends on lane / 16 only, so
        // chunk i (row + 64 i) has the same 16-byte position
        const int cid = wave * 64 + lane;  // 16-byte chunk id in the A tile
        const int row = cid >> 2, pos = cid & 3;
        const uint32_t q16 = (uint32_t)((pos ^ a_swizzle<4>(row)) * 16);
        o.a0 = GATHER ? q16 : (uint32_t)row * K + q16;
    }
    {
        // chunk 0: stage row wave * 4 + lane / 16; the swizzle key row & 7 is the same for
        // chunk i (row + 16 i)
        const int cid = wave * 64 + lane;
        const int row = cid >> 4, pos = cid & 15;
        const int c = pos ^ ((row & 7) << 1);  // logical 16-column chunk (SW: gate c < 8, else up)
        if constexpr (SW) {
            // past H (the last column tile when H % 128 != 0) these read other columns; their
            // weight scales are 0, so those activations are 0 and never stored
            const uint32_t j = 16 * (c & 7);
            o.b0 = (uint32_t)row * o.n + (c < 8 ? j : (uint32_t)a.epi.H + j);
        } else {
            o.b0 = (uint32_t)row * o.n + (uint32_t)(16 * c);
        }
    }
    return o;
}

// The plan of row tile (g, m0, vrows) x column tile nt.  The weight resource starts at the tile's
// first gate column: a weight row k >= K then lies past its end (the resource is nt * 128 bytes
// shorter), and so does no valid column of row K - 1 (nt * 128 + 128 <= H, or the columns are
// past H).
template <bool GATHER>
__device__ __forceinline__ PfSrc pf_src(const GemmArgs& a, const int g, const int m0, const int vrows, const int nt,
                                        const int wave, const int lane)
{
    PfSrc s;
    const int64_t K = a.K;
    s.ares = GATHER ? make_rsrc(a.x, (uint32_t)(a.x_rows * K))
                    : make_rsrc(a.x + (int64_t)m0 * K, (uint32_t)((int64_t)(vrows < 256 ? vrows : 256) * K));
    const int64_t c0 = (int64_t)nt * 128;
    s.bres = make_rsrc(a.w + (int64_t)g * a.w_gstride + c0, (uint32_t)(K * a.N - c0));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        s.ga[i] = 0x80000000u;
        if constexpr (GATHER) {
            const int row = ((i * 4 + wave) * 64 + lane) >> 2;
            const int srow = row < vrows ? src_row(a, m0 + row) : -1;
            if (srow >= 0) s.ga[i] = (uint32_t)srow * (uint32_t)K;
        }
    }
    return s;
}

// A plan that fetches nothing: the stage stream past a workgroup's last tile.
__device__ __forceinline__ PfSrc pf_dead(const GemmArgs& a)
{
    PfSrc s;
    s.ares = make_rsrc(a.x, 0u);
    s.bres = make_rsrc(a.w, 0u);
#pragma unroll
    for (int i = 0; i < 4; ++i) s.ga[i] = 0x80000000u;
    return s;
}

// DMA chunk I of stage kt into ring slot `slot` (I < 4: activation chunk I, else weight chunk
// I - 4).  CHECK: stages past K fetch nothing (activation offsets would run into the next rows;
// weight offsets already lie outside their resource).
template <int I, bool GATHER, bool CHECK>
__device__ __forceinline__ void pf_dma(const PfSrc& s, const PfOffs& o, const int kt, const int nk, const int slot,
                                       const uint32_t lds_base, const int wave)
{
    using C = PfCfg;
    const uint32_t sa = lds_base + (uint32_t)(slot * C::STAGE);
    if constexpr (I < 4) {
        uint32_t off = (GATHER ? s.ga[I] + o.a0 : o.a0) + ((uint32_t)I * o.ka + (uint32_t)(kt * C::BK));
        if (CHECK && kt >= nk) off = 0x80000000u;
        dma16(s.ares, off, __builtin_amdgcn_readfirstlane(sa + (uint32_t)((I * 4 + wave) * 1024)));
    } else {
        dma16(s.bres, o.b0 + (uint32_t)((I - 4) * 16 + kt * C::BK) * o.n,
              __builtin_amdgcn_readfirstlane(sa + C::A_BYTES + (uint32_t)(((I - 4) * 4 + wave) * 1024)));
    }
}

// LDS map (bytes): the ring, then two scale slots (alternate tiles), each the per-row activation
// scales [256] and per-column weight scales [256] (128 gate then 128 up), row maxima of the two
// column-half waves [2][256], 127 / amax [256], the round-order table.
constexpr int kPfRing = PfCfg::STAGES_ * PfCfg::STAGE;
constexpr int kPfSc = kPfRing, kPfScSlot = 2048, kPfRm = kPfSc + 2 * kPfScSlot, kPfInv = kPfRm + 2048;
constexpr int kPfOrd = kPfInv + 1024;
constexpr int kPfFlag = kPfOrd + 3 * 4 * (CB_MAX_EXPERTS + 1);  // the deferred requant's exchange outcome
constexpr int kPfLds = kPfFlag + 16;
static_assert(PfCfg::A_ISSUE == 4 && PfCfg::B_ISSUE == 4 && PfCfg::NW == 4 && PfCfg::FM == 4 && PfCfg::FN == 4,
              "the stage schedule below is written for this configuration");

// Exchange groups of the persistent grid: RT consecutive row tiles x all ntl column tiles.
struct PfPlace {
    int slot, rt, nt, slots, RT;
};

__device__ __forceinline__ PfPlace pf_place(int ntl, int grid, int b)
{
    PfPlace p;
    if (ntl == 16 && grid == 256) {
        // Workgroup b is dispatched to XCD b % 8.  Slot s = the XCD pair (2 s, 2 s + 1): its 64
        // workgroups hold the slot's 4 row tiles x all 16 column tiles, column tiles 0-7 on the
        // even XCD and 8-15 on the odd one (before the per-round rotation).  Each XCD then streams
        // half of a heavy expert's weight for 4 row tiles, where one XCD per 2 row tiles streamed
        // all of it: the weight bytes fetched from HBM per heavy row tile halve, for twice the
        // activation fetches (each row tile's activation slab goes to two L2s).  Measured, same
        // box, interleaved: Zipf 4.04-4.07 ms against 4.07-4.12 with one XCD per 2 row tiles x 16
        // column tiles; XCD quads (8 row tiles x 4 column tiles per XCD) 4.08-4.10, all 8 XCDs
        // (16 x 2) 4.18-4.20.
        const int x = b & 7, j = b >> 3;
        p.slot = x >> 1;
        p.rt = j >> 3;
        p.nt = 8 * (x & 1) + (j & 7);
        p.slots = 4;
        p.RT = 4;
    } else {
        p.slot = b / ntl;
        p.rt = 0;
        p.nt = b % ntl;
        p.slots = grid / ntl;
        p.RT = 1;
    }
    return p;
}

// Round order of the row tiles.  Row tiles of experts with more than 256 rows ("heavy": they reuse
// every weight slab, so they are MFMA-bound) and those of experts with at most 256 rows ("light":
// one tile reads its expert's whole weight once, HBM-bound) are grouped into rounds of RT tiles of
// one kind, and the two kinds of rounds are interleaved in proportion, so that while most exchange
// groups multiply, some stream weights.  The per-expert prefix counts live in LDS.
struct PfOrder {
    int n_heavy, n_light;  // row tiles of each kind
    int heavy_rounds, light_rounds;
};

// LDS table: heavy tile prefix [E + 1], light tile prefix [E + 1], first tile [E + 1] per expert.
constexpr int kPfOrdE = CB_MAX_EXPERTS + 1;

__device__ PfOrder pf_build_order(const GroupTable& gt, int RT, CB_LDS int* tab)
{
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    CB_LDS int* hp = tab;
    CB_LDS int* lp = tab + kPfOrdE;
    CB_LDS int* ts = tab + 2 * kPfOrdE;
    static_assert(CB_MAX_EXPERTS == 256, "one thread per expert");
    const int t0 = gt.tile_start[t], n = gt.tile_start[t + 1] - t0;
    int lt = n == 1 ? 1 : 0, ht = n == 1 ? 0 : n;
    // inclusive scan of (lt, ht) over the 256 threads: within each wave, then across the 4 waves
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int l2 = __shfl_up(lt, o, 64), h2 = __shfl_up(ht, o, 64);
        if (lane >= o) {
            lt += l2;
            ht += h2;
        }
    }
    __shared__ int wtot[2][4];
    if (lane == 63) {
        wtot[0][wave] = lt;
        wtot[1][wave] = ht;
    }
    __syncthreads();
    for (int w = 0; w < wave; ++w) {
        lt += wtot[0][w];
        ht += wtot[1][w];
    }
    lp[t + 1] = lt;
    hp[t + 1] = ht;
    ts[t] = t0;
    if (t == 0) {
        lp[0] = 0;
        hp[0] = 0;
        ts[CB_MAX_EXPERTS] = gt.tile_start[CB_MAX_EXPERTS];
    }
    __syncthreads();
    PfOrder o;
    o.n_light = lp[CB_MAX_EXPERTS];
    o.n_heavy = hp[CB_MAX_EXPERTS];
    o.heavy_rounds = (o.n_heavy + RT - 1) / RT;
    o.light_rounds = (o.n_light + RT - 1) / RT;
    return o;
}

// A row tile: its index, group, first row and valid rows (mt = -1: none).
struct PfTile {
    int mt, g, m0, vrows;
};

// The i-th row tile of one kind (i < its count), in expert order: expert g = the first with
// prefix[g + 1] > i.
__device__ __forceinline__ PfTile pf_kth_tile(const GroupTable& gt, const CB_LDS int* tab, bool light, int i)
{
    const CB_LDS int* pre = tab + (light ? kPfOrdE : 0);
    int lo = 0, hi = CB_MAX_EXPERTS - 1;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (pre[mid + 1] > i) hi = mid;
        else lo = mid + 1;
    }
    PfTile t;
    const int j = i - pre[lo];  // tile j of group lo
    t.g = __builtin_amdgcn_readfirstlane(lo);
    t.mt = __builtin_amdgcn_readfirstlane(tab[2 * kPfOrdE + lo] + j);
    t.m0 = (t.g ? gt.row_end[t.g - 1] : 0) + j * 256;
    t.vrows = gt.row_end[t.g] - t.m0;
    return t;
}

// Row tile of position rt in round q (mt = -1: past the last tile of the round's kind).
__device__ __forceinline__ PfTile pf_round_tile(const GroupTable& gt, const CB_LDS int* tab, const PfOrder& o, int RT,
                                                int q, int rt)
{
    PfTile none;
    none.mt = -1;
    none.g = none.m0 = none.vrows = 0;
    const int T = o.heavy_rounds + o.light_rounds;
    if (q >= T) return none;
    // round q is light when the proportional count of light rounds steps at q
    const int lq = (int)(((int64_t)(q + 1) * o.light_rounds) / T), lq0 = (int)(((int64_t)q * o.light_rounds) / T);
    const bool light = lq > lq0;
    const int idx = (light ? lq0 : q - lq0) * RT + rt;
    if (idx >= (light ? o.n_light : o.n_heavy)) return none;
    return pf_kth_tile(gt, tab, light, idx);
}

// Tile mt in natural order (the fix-up launch).
__device__ __forceinline__ PfTile pf_tile_at(const GroupTable& gt, int mt)
{
    PfTile t;
    t.mt = mt;
    t.g = group_of_tile(gt, mt);
    t.m0 = (t.g ? gt.row_end[t.g - 1] : 0) + (mt - gt.tile_start[t.g]) * 256;
    t.vrows = gt.row_end[t.g] - t.m0;
    return t;
}

__device__ __forceinline__ int pf_total_rounds(const PfOrder& o) { return o.heavy_rounds + o.light_rounds; }

// ---- the K loop ------------------------------------------------------------------------------
// The plan of stage st of the stream: this tile's, or past K (PF) the next tile's (stage st - nk).
// Value selects, not control flow, so the scheduled loop body stays one block.
template <bool PF>
__device__ __forceinline__ PfSrc pf_stream(const PfSrc& cur, const PfSrc& nxt, const int st, const int nk, int& lst)
{
    if constexpr (!PF) {
        lst = st;
        return cur;
    } else {
        const bool n = st >= nk;
        lst = n ? st - nk : st;
        PfSrc s;
        s.ares = n ? nxt.ares : cur.ares;
        s.bres = n ? nxt.bres : cur.bres;
#pragma unroll
        for (int i = 0; i < 4; ++i) s.ga[i] = n ? nxt.ga[i] : cur.ga[i];
        return s;
    }
}

// Ring slot of stage kt: (rb + kt) % 4.  With PF (nk >= 4) the stages past this tile's K are the
// next tile's first 3.5 stages (its prologue), so the next tile starts at ring slot (rb + nk) % 4
// with its stages already in flight; nxt is a dead plan when there is no next tile.  Without PF
// they fetch nothing.
template <int NV, bool PF, bool GATHER>
__device__ __forceinline__ void pf_kloop(const PfSrc& dma, const PfSrc& nxt, const PfOffs& offs, const int nk,
                                         const int rb, uint8_t* smem,
                                         const uint32_t (&a_rd)[4][2], const uint32_t (&b_rd)[4], v16i (&acc)[4][4],
                                         const int wave, const bool first)
{
    using C = PfCfg;
    constexpr int NVA = NV > 0 ? NV : 1;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(CB_LDS uint8_t*)smem;
    const CB_LDS uint8_t* sm = (const CB_LDS uint8_t*)smem;
    v4i a0[NVA], a1[NVA], b0[4], b1[4];
    auto rdb = [&](int kt, int ks, int fn, v4i (&bf)[4]) {
        const CB_LDS uint8_t* base = sm + ((rb + kt) & 3) * C::STAGE + C::A_BYTES;
        const uint32_t o = b_rd[fn] + (uint32_t)(ks * 32 * C::BN);
        const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((CB_LDS v2i*)(base + o));
        const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((CB_LDS v2i*)(base + o + 8 * C::BN));
        bf[fn] = v4i{lo[0], lo[1], hi[0], hi[1]};
    };
    auto rda = [&](int kt, int ks, int fm, v4i (&af)[NVA]) {
        // a_rd[fm][ks] = a_rd[0][ks] + fm * 64 rows (the swizzle depends on the row within its
        // 32-row block only): an instruction immediate
        if (fm < NV)
            af[fm < NVA ? fm : 0] = *(const CB_LDS v4i*)(sm + ((rb + kt) & 3) * C::STAGE + a_rd[0][ks] + fm * 64 * C::BK);
    };
    // ZERO: the tile's first MFMAs, which start from a zero accumulator (no separate clearing of
    // the 256 accumulator registers)
    auto mrow = [&](auto fm_t, const v4i (&af)[NVA], const v4i (&bf)[4], auto zero_t) {
        constexpr int fm = decltype(fm_t)::value;
        constexpr bool ZERO = decltype(zero_t)::value;
        if constexpr (fm < NV) {
#pragma unroll
            for (int fn = 0; fn < 4; ++fn)
                acc[fm][fn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[fm < NVA ? fm : 0], bf[fn],
                                                                    ZERO ? v16i{} : acc[fm][fn], 0, 0, 0);
        }
    };
    // one chunk: a DMA, then its fragment reads interleaved one for one with 4 MFMAs; chunks are
    // fenced from each other so the DMAs stay spread over the half-step
    auto fence = [&]() {
        if constexpr (NV > 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // stage 0 landed: the first tile of a workgroup waits for its DMAs; a later tile's prologue was
    // drained by its predecessor's epilogue (every VMEM result waited for before its exchange), so
    // only the barrier
    if (first) wait_vmcnt_barrier<2 * C::ISSUE + C::A_ISSUE>();
    else wait_vmcnt_barrier<63>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0) in the compiler's own accounting
    if constexpr (NV > 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) rdb(0, 0, c, b0);
#pragma unroll
        for (int c = 0; c < 4; ++c) rda(0, 0, c, a0);
    }
    using F = std::integral_constant<bool, false>;
    using T = std::integral_constant<bool, true>;
    // half 1 of iteration kt: MFMAs of step 0 (a0/b0), reads of step 1, the B chunks of stage kt + 3
    auto half1 = [&](const int kt, auto zero_t) {
        int sb;
        const PfSrc db = pf_stream<PF>(dma, nxt, kt + 3, nk, sb);
        const int s3 = (rb + kt + 3) & 3;
        pf_dma<4, GATHER, !PF>(db, offs, sb, nk, s3, lds_base, wave);
        if constexpr (NV > 0) { rdb(kt, 1, 0, b1); rdb(kt, 1, 1, b1); }
        mrow(std::integral_constant<int, 0>(), a0, b0, zero_t);
        fence();
        pf_dma<5, GATHER, !PF>(db, offs, sb, nk, s3, lds_base, wave);
        if constexpr (NV > 0) { rdb(kt, 1, 2, b1); rdb(kt, 1, 3, b1); }
        mrow(std::integral_constant<int, 1>(), a0, b0, zero_t);
        fence();
        pf_dma<6, GATHER, !PF>(db, offs, sb, nk, s3, lds_base, wave);
        rda(kt, 1, 0, a1);
        rda(kt, 1, 1, a1);
        mrow(std::integral_constant<int, 2>(), a0, b0, zero_t);
        fence();
        pf_dma<7, GATHER, !PF>(db, offs, sb, nk, s3, lds_base, wave);
        rda(kt, 1, 2, a1);
        rda(kt, 1, 3, a1);
        mrow(std::integral_constant<int, 3>(), a0, b0, zero_t);
        fence();
    };
    // half 2 of iteration kt: stage kt + 1 landed (outstanding: stage kt + 2 and kt + 3) and stage
    // kt fully read; MFMAs of step 1 (a1/b1), reads of stage kt + 1 step 0, the A chunks of stage
    // kt + 4 into the slot stage kt just left
    auto half2 = [&](const int kt) {
        wait_vmcnt_barrier<2 * C::ISSUE>();
        int sa;
        const PfSrc da = pf_stream<PF>(dma, nxt, kt + 4, nk, sa);
        const int s4 = (rb + kt) & 3;
        pf_dma<0, GATHER, !PF>(da, offs, sa, nk, s4, lds_base, wave);
        if constexpr (NV > 0) { rdb(kt + 1, 0, 0, b0); rdb(kt + 1, 0, 1, b0); }
        mrow(std::integral_constant<int, 0>(), a1, b1, F());
        fence();
        pf_dma<1, GATHER, !PF>(da, offs, sa, nk, s4, lds_base, wave);
        if constexpr (NV > 0) { rdb(kt + 1, 0, 2, b0); rdb(kt + 1, 0, 3, b0); }
        mrow(std::integral_constant<int, 1>(), a1, b1, F());
        fence();
        pf_dma<2, GATHER, !PF>(da, offs, sa, nk, s4, lds_base, wave);
        rda(kt + 1, 0, 0, a0);
        rda(kt + 1, 0, 1, a0);
        mrow(std::integral_constant<int, 2>(), a1, b1, F());
        fence();
        pf_dma<3, GATHER, !PF>(da, offs, sa, nk, s4, lds_base, wave);
        rda(kt + 1, 0, 2, a0);
        rda(kt + 1, 0, 3, a0);
        mrow(std::integral_constant<int, 3>(), a1, b1, F());
        fence();
    };
    // fragments without valid rows get no MFMAs: their accumulators are plain zeros
#pragma unroll
    for (int fm = NV; fm < 4; ++fm)
#pragma unroll
        for (int fn = 0; fn < 4; ++fn) acc[fm][fn] = v16i{};
    // the loop rotated by half an iteration, so that the tile's first half-step (the MFMAs from a
    // zero accumulator) stands outside it
    half1(0, T());
#pragma nounroll
    for (int kt = 0; kt < nk - 1; ++kt) {
        half2(kt);
        half1(kt + 1, F());
    }
    half2(nk - 1);
}

// Prologue of a tile: stages 0-2 and the A chunks of stage 3 (the loop issues the rest).
template <bool GATHER>
__device__ __forceinline__ void pf_prologue(const PfSrc& s, const PfOffs& o, const int nk, uint8_t* smem,
                                            const int wave)
{
    const uint32_t lds_base = (uint32_t)(uintptr_t)(CB_LDS uint8_t*)smem;
#pragma unroll
    for (int st = 0; st < 3; ++st) {
        pf_dma<0, GATHER, true>(s, o, st, nk, st, lds_base, wave);
        pf_dma<1, GATHER, true>(s, o, st, nk, st, lds_base, wave);
        pf_dma<2, GATHER, true>(s, o, st, nk, st, lds_base, wave);
        pf_dma<3, GATHER, true>(s, o, st, nk, st, lds_base, wave);
        pf_dma<4, GATHER, true>(s, o, st, nk, st, lds_base, wave);
        pf_dma<5, GATHER, true>(s, o, st, nk, st, lds_base, wave);
        pf_dma<6, GATHER, true>(s, o, st, nk, st, lds_base, wave);
        pf_dma<7, GATHER, true>(s, o, st, nk, st, lds_base, wave);
    }
    pf_dma<0, GATHER, true>(s, o, 3, nk, 3, lds_base, wave);
    pf_dma<1, GATHER, true>(s, o, 3, nk, 3, lds_base, wave);
    pf_dma<2, GATHER, true>(s, o, 3, nk, 3, lds_base, wave);
    pf_dma<3, GATHER, true>(s, o, 3, nk, 3, lds_base, wave);
}

// Scales of a tile, fetched into registers: thread t takes tile row t's activation scale (the row
// clamped into the group, through the row index when gathered) and tile column t's weight scale
// (128 gate then 128 up columns; 0 past H).
struct PfScales {
    float xs, cs;
};

__device__ __forceinline__ PfScales pf_scales(const GemmArgs& a, const PfTile& t, int nt)
{
    const int tid = opaque((int)threadIdx.x);  // per-tile address math stays in the tile
    const int g = t.g, m0 = t.m0, r1 = t.m0 + t.vrows;
    const int xr = m0 + tid;
    PfScales s;
    s.xs = src_x_scale(a, xr < r1 ? xr : r1 - 1);
    const int64_t H = a.epi.H, N = a.N;
    const int64_t jc = (int64_t)nt * 128 + (tid & 127);
    const int64_t wc = tid < 128 ? jc : H + jc;
    const __amdgpu_buffer_rsrc_t wsr = make_rsrc(a.epi.w_scale + (int64_t)g * N, (uint32_t)(N * 4));
    s.cs = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wsr, jc < H ? (uint32_t)(wc * 4) : 0x80000000u, 0, 0));
    return s;
}

// Per-lane LDS read offsets of the fragments (stage-relative).  A: fragment fm of wave row wm
// covers tile rows (2 fm + wm) * 32 + lane % 32, k chunk 2 ks + lane / 32.  B: the transposing
// read of gemm_lds.hpp (one base offset per fragment, the rest are instruction immediates).
__device__ __forceinline__ void pf_read_offsets(int wm, int wn, int lane, uint32_t (&a_rd)[4][2], uint32_t (&b_rd)[4])
{
    using C = PfCfg;
#pragma unroll
    for (int fm = 0; fm < 4; ++fm) {
        const int r = (2 * fm + wm) * 32 + (lane & 31);
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int q = 2 * ks + (lane >> 5);
            a_rd[fm][ks] = (uint32_t)(r * C::BK + ((q ^ a_swizzle<C::ACH>(r)) << 4));
        }
    }
    const int gq = lane >> 4, s = lane & 15;
#pragma unroll
    for (int fn = 0; fn < 4; ++fn) {
        // fragments 0, 1: gate columns wn * 64 + 32 fn; 2, 3: the matching up columns (+128)
        const int tcol = (fn < 2 ? 0 : 128) + wn * 64 + (fn & 1) * 32;
        const int cc = (tcol >> 4) + (gq & 1);
        const int row = (gq >> 1) * 16 + (s >> 1);
        const int pos = cc ^ ((s >> 1) << 1);
        b_rd[fn] = (uint32_t)(row * C::BN + pos * 16 + (s & 1) * 8);
    }
}

// Accumulator element read into a VGPR, in program order: the compiler would otherwise move all
// 256 accumulators into VGPRs at the start of the epilogue and spill everything else.
__device__ __forceinline__ int acc_read(int v)
{
    int r;
    asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(r) : "a"(v));
    return r;
}

// A value moved to / read back from an accumulator register (the epilogue's storage).
__device__ __forceinline__ float to_agpr(float v)
{
    float r;
    asm("v_accvgpr_write_b32 %0, %1" : "=a"(r) : "v"(v));
    return r;
}

__device__ __forceinline__ float from_agpr(float v)
{
    float r;
    asm("v_accvgpr_read_b32 %0, %1" : "=v"(r) : "a"(v));
    return r;
}

// One step of a half-wave max over non-negative float bit patterns held as u32 (integer max needs
// no NaN canonicalisation).  The DPP move with a zero old value and bound_ctrl folds into the max:
// one v_max_u32_dpp per step.  Lanes outside ROWS see 0 and keep their own value.
template <int CTRL, int ROWS>
__device__ __forceinline__ u32 umax_dpp(u32 v)
{
    const u32 o = (u32)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWS, 0xF, true);
    return v > o ? v : o;
}

// rint16 for the requant's products v = act * (127 / amax) of one row: fp16 rounding
// (v_cvt_f16_f32), fp16 round-half-even, fp16 -> int16 (NaN -> 0).  |act| <= amax for every act of
// the row (amax is their maximum, NaN ignored), so |v| <= 127 (1 + 2^-23) and the fp16 value lies
// in [-127, 127]: rint16's clamp to [-128, 127] never acts and is left out.  Only the low byte of
// the result is used.
__device__ __forceinline__ int rint16_h(float v)
{
    // opaque: v is the rounded fp32 product, not folded into a mixed-precision fma with one rounding
    const _Float16 r = __builtin_elementwise_roundeven((_Float16)opaque(v));
    int i;
    asm("v_cvt_i16_f16 %0, %1" : "=v"(i) : "v"(r));
    return i;
}

// The exchange wait of one thread: poll the counter until it reaches target, at most spin_limit
// times (a negative limit, the test hook, gives up at once).  Once any wait of the call has given
// up (the status word is set, e.g. because CUs held by other work keep part of the grid from
// running), every later wait gives up at once too, so the call stalls for one wait at most and
// the fix-up launch computes the rest.  Returns 0 when it gave up.
__device__ __forceinline__ u32 pf_wait(const EpiArgs& e, u32* counter, const u32 target)
{
    if (e.spin_limit < 0) return 0u;
    for (int spins = 0; __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target; ++spins) {
        if (spins >= e.spin_limit ||
            ((spins & 255) == 0 && (__hip_atomic_load(e.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 1u)))
            return 0u;
        __builtin_amdgcn_s_sleep(8);
    }
    // the counter reached its target: the row maxima published before those arrivals (release) are
    // visible to this thread, and through the barrier that follows to the whole workgroup
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return 1u;
}

// Publishing side of the exchange, executed by every thread after its row-maximum atomics and
// followed by a barrier, after which thread 0 adds the workgroup's arrival (pf_arrive).  The maxima
// and the counters are touched only by agent-scope atomics, which gfx950 performs at the device's
// coherence point, beyond the XCD's non-coherent L2; `s_waitcnt vmcnt(0)` returns once every vector
// memory operation of the wave has completed, its returning and non-returning atomics included,
// so after each wave's wait and the barrier, every maximum of the tile is performed before the
// arrival is issued.  The waiting side reads the counter and the maxima with agent-scope atomic
// loads and takes an agent-scope acquire fence once the count is complete (pf_wait).
// A release written in the memory model instead (a release fence per wave and a release add)
// compiles to `buffer_wbl2 sc1`, a write-back of the XCD's whole L2, five times per tile: measured
// 4.06 -> 5.14 ms per prefill call.  The wait also drains the next tile's stage DMAs, which the
// K loop's first wait relies on.
__device__ __forceinline__ void pf_release_maxima() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ void pf_arrive(u32* counter)
{
    __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Four int8 values of one row (consecutive columns) at a dword offset of y: one dword store, or
// four byte stores when y itself is not 4-byte aligned (H % 16 == 0 keeps every row and column
// offset a multiple of 4, so the choice is uniform).
__device__ __forceinline__ void pf_store4(const u32 v, const __amdgpu_buffer_rsrc_t yr, const uint32_t off, const bool bytes)
{
    if (bytes) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(v >> (8 * i)), yr, off == 0x80000000u ? off : off + i, 0, 0);
    } else {
        __builtin_amdgcn_raw_buffer_store_b32((int)v, yr, off, 0, 0);
    }
}

// One persistent GMSQ tile after its K loop: everything from the SwiGLU to the int8 stores.
// Returns false when the exchange wait timed out (the tile stored nothing and is marked for the
// fix-up launch).
template <bool FIXUP>
__device__ __forceinline__ void pf_epilogue(const GemmArgs& a, uint8_t* smem, v16i (&acc)[4][4], const PfTile& t,
                                            const int nt, const int par, const int arr_idx, const u32 arr_target,
                                            const int tile_id)
{
    // opaque: the per-tile address math is recomputed here rather than hoisted out of the tile loop
    // (and spilled across the K loop)
    const int tid = opaque((int)threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const EpiArgs& e = a.epi;
    const int64_t H = e.H;
    const int m0 = t.m0, vrows = t.vrows;
    const CB_LDS float* xs_l = (const CB_LDS float*)((CB_LDS uint8_t*)smem + kPfSc + par * kPfScSlot);
    const CB_LDS float* cs_l = xs_l + 256;
    CB_LDS float* rm_l = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfRm);
    CB_LDS float* inv_l = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfInv);

    // Nothing to wait for first: the ring's slots already take the next tile's first stages, and
    // this tile's scales are in LDS slot par since before its K loop.
    // 1. SwiGLU.  Lane (h = lane / 32, c = lane % 32) of fragment (fm, fn) holds rows
    //    (2 fm + wm) * 32 + 8 (r / 4) + 4 h + r % 4 (r = 0..15), column c of the fragment.
    const int h = lane >> 5, c = lane & 31;
    float wsg[2], wsu[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        wsg[j] = cs_l[wn * 64 + j * 32 + c];
        wsu[j] = cs_l[128 + wn * 64 + j * 32 + c];
    }
    // the 128 activations of a lane are parked in accumulator registers (freed by the SwiGLU
    // inputs as they are consumed) until the final row maxima are known
    float act[4][2][16];
#pragma unroll
    for (int fm = 0; fm < 4; ++fm) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int row = (2 * fm + wm) * 32 + 8 * q + 4 * h;
            const v4f xs4 = *(const CB_LDS v4f*)(xs_l + row);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    act[fm][j][4 * q + i] = to_agpr(swiglu((float)acc_read(acc[fm][j][4 * q + i]),
                                                           (float)acc_read(acc[fm][j + 2][4 * q + i]), xs4[i], wsg[j],
                                                           wsu[j]));
        }
    }
    // row maxima of this wave's 64 act columns, then of the two waves sharing the rows (LDS).  A
    // NaN activation is ignored (a NaN bit pattern counts as 0), like the reference's compare-based
    // maximum; the 64 row values of a lane are reduced step by step together so that the DPP
    // steps of different rows interleave.
    if (!FIXUP) {
        u32 m[4][16];
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const u32 u0 = __float_as_uint(from_agpr(act[fm][0][r])) & 0x7fffffffu;
                const u32 u1 = __float_as_uint(from_agpr(act[fm][1][r])) & 0x7fffffffu;
                const u32 v0 = u0 > 0x7f800000u ? 0u : u0, v1 = u1 > 0x7f800000u ? 0u : u1;
                m[fm][r] = v0 > v1 ? v0 : v1;
            }
        // row_ror 1, 2, 4, 8 within each 16-lane row, then row_bcast:15 into rows 1 and 3: lanes
        // 16..31 and 48..63 end with their half-wave's maximum
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) m[fm][r] = umax_dpp<0x121, 0xF>(m[fm][r]);
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) m[fm][r] = umax_dpp<0x122, 0xF>(m[fm][r]);
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) m[fm][r] = umax_dpp<0x124, 0xF>(m[fm][r]);
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) m[fm][r] = umax_dpp<0x128, 0xF>(m[fm][r]);
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
            for (int r = 0; r < 16; ++r) m[fm][r] = umax_dpp<0x142, 0xA>(m[fm][r]);
        if (c == 16) {
#pragma unroll
            for (int fm = 0; fm < 4; ++fm)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *(CB_LDS v4i*)(rm_l + wn * 256 + (2 * fm + wm) * 32 + 8 * q + 4 * h) =
                        v4i{(int)m[fm][4 * q], (int)m[fm][4 * q + 1], (int)m[fm][4 * q + 2], (int)m[fm][4 * q + 3]};
        }
        __syncthreads();
        if (tid < vrows) {
            const u32 m0v = __float_as_uint(rm_l[tid]), m1v = __float_as_uint(rm_l[256 + tid]);
            __hip_atomic_fetch_max(e.amax + m0 + tid, m0v > m1v ? m0v : m1v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        // 2. exchange: every row maximum of this tile is released before the arrival count
        pf_release_maxima();
        __syncthreads();
        if (tid == 0) {
            pf_arrive(e.arrive + arr_idx);
            const u32 ok = pf_wait(e, e.arrive + arr_idx, arr_target);
            if (!ok) {
                // this tile's y waits for the fix-up launch
                __hip_atomic_fetch_or(e.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(e.redo + tile_id, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            rm_l[0] = __uint_as_float(ok);
        }
        __syncthreads();
        const bool ok = __float_as_uint(rm_l[0]) != 0;
        if (!ok) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            return;
        }
    }

    // 3. final row maxima -> 127 / amax through LDS; the nt = 0 tile writes y_scale
    {
        float am = 0.0f;
        if (tid < vrows) am = __uint_as_float(__hip_atomic_load(e.amax + m0 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (!(am > kFltMin)) am = kFltMin;
        inv_l[tid] = 127.0f / am;
        if (nt == 0 && tid < vrows) e.yq_scale[m0 + tid] = am * kInv127;
        // every VMEM result (the next tile's first stages included) is in before the stores below,
        // so the next tile's loop starts without a vmcnt wait
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
    }
    const __amdgpu_buffer_rsrc_t yr = make_rsrc(e.yq + (int64_t)m0 * H, (uint32_t)((int64_t)(vrows < 256 ? vrows : 256) * H));
    const int qi = c & 3;  // position in the lane quad
#pragma unroll
    for (int fm = 0; fm < 4; ++fm) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int row = (2 * fm + wm) * 32 + 8 * q + 4 * h;
            const v4f inv4 = *(const CB_LDS v4f*)(inv_l + row);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                // this lane: rows row..row+3 of column c; clamp-and-narrow == saturating rint16,
                // an all-zero row gives 0 * inf = NaN -> 0
                const u32 x = pack4_i8(rint16_h(from_agpr(act[fm][j][4 * q + 0]) * inv4[0]),
                                       rint16_h(from_agpr(act[fm][j][4 * q + 1]) * inv4[1]),
                                       rint16_h(from_agpr(act[fm][j][4 * q + 2]) * inv4[2]),
                                       rint16_h(from_agpr(act[fm][j][4 * q + 3]) * inv4[3]));
                // 4 x 4 byte transpose across the quad: lane qi ends with row row + qi, columns
                // (c & ~3) .. +3.  Step 1 swaps 16-bit halves with lane qi ^ 2, step 2 bytes with qi ^ 1.
                const u32 p = (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);
                const u32 z = (qi & 2) ? __builtin_amdgcn_perm(x, p, 0x07060302u) : __builtin_amdgcn_perm(p, x, 0x05040100u);
                const u32 pz = (u32)__builtin_amdgcn_update_dpp(0, (int)z, 0xB1, 0xF, 0xF, false);
                const u32 y = (qi & 1) ? __builtin_amdgcn_perm(pz, z, 0x03070105u) : __builtin_amdgcn_perm(pz, z, 0x06020400u);
                const int64_t col = (int64_t)nt * 128 + wn * 64 + j * 32 + (c & ~3);
                const uint32_t off = col < H ? (uint32_t)((row + qi) * H + col) : 0x80000000u;
                pf_store4(y, yr, off, ((uintptr_t)e.yq & 3) != 0);
            }
        }
    }
}

// The deferred requant: a tile's activations stay in VGPRs after its epilogue has published the
// row maxima, through the workgroup's whole next K loop; after that loop the row tile's exchange
// has long completed, and the previous tile is requantised and stored before the current one is
// published.  No workgroup waits for its row tile's other column tiles, so a late one (a slow
// weight line, an HBM-bound tile of a small expert) costs nothing until it is a whole tile late.
//
// publish (after the K loop): SwiGLU from the accumulators into act, row maxima of |act| across
// the lanes (DPP) and the two waves sharing the rows (LDS), one agent-scope atomicMax per (row,
// tile), then one arrival on the row tile's counter once every maximum has completed.
__device__ __forceinline__ void pf_publish(const GemmArgs& a, uint8_t* smem, v16i (&acc)[4][4], const PfTile& t,
                                           const int par, float (&act)[4][2][16])
{
    const int tid = opaque((int)threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const EpiArgs& e = a.epi;
    const CB_LDS float* xs_l = (const CB_LDS float*)((CB_LDS uint8_t*)smem + kPfSc + par * kPfScSlot);
    const CB_LDS float* cs_l = xs_l + 256;
    CB_LDS float* rm_l = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfRm);
    const int h = lane >> 5, c = lane & 31;
    float wsg[2], wsu[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        wsg[j] = cs_l[wn * 64 + j * 32 + c];
        wsu[j] = cs_l[128 + wn * 64 + j * 32 + c];
    }
    // The activations are built in the accumulator registers the SwiGLU inputs free (the 128
    // VGPRs they occupy during the next K loop are then not needed on top of this step's own), and
    // moved to VGPRs at the end.
    // lane (h, c) of fragment (fm, fn) holds rows (2 fm + wm) * 32 + 8 (r / 4) + 4 h + r % 4, column c
#pragma unroll
    for (int fm = 0; fm < 4; ++fm) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int row = (2 * fm + wm) * 32 + 8 * q + 4 * h;
            const v4f xs4 = *(const CB_LDS v4f*)(xs_l + row);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    act[fm][j][4 * q + i] = to_agpr(swiglu((float)acc_read(acc[fm][j][4 * q + i]),
                                                           (float)acc_read(acc[fm][j + 2][4 * q + i]), xs4[i], wsg[j], wsu[j]));
        }
    }
    // |act| as u32 bit patterns, NaN counted as 0 (the reference's compare-based maximum ignores
    // it); one fragment row at a time (16 values per lane), so that the maxima do not add 64
    // registers to the 128 activations held here.  row_ror 1, 2, 4, 8 within each 16-lane row, then
    // row_bcast:15 into rows 1 and 3: lanes 16..31 and 48..63 end with their half-wave's maximum.
#pragma unroll
    for (int fm = 0; fm < 4; ++fm) {
        u32 m[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const u32 u0 = __float_as_uint(from_agpr(act[fm][0][r])) & 0x7fffffffu;
            const u32 u1 = __float_as_uint(from_agpr(act[fm][1][r])) & 0x7fffffffu;
            const u32 v0 = u0 > 0x7f800000u ? 0u : u0, v1 = u1 > 0x7f800000u ? 0u : u1;
            m[r] = v0 > v1 ? v0 : v1;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) m[r] = umax_dpp<0x121, 0xF>(m[r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) m[r] = umax_dpp<0x122, 0xF>(m[r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) m[r] = umax_dpp<0x124, 0xF>(m[r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) m[r] = umax_dpp<0x128, 0xF>(m[r]);
#pragma unroll
        for (int r = 0; r < 16; ++r) m[r] = umax_dpp<0x142, 0xA>(m[r]);
        if (c == 16) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *(CB_LDS v4i*)(rm_l + wn * 256 + (2 * fm + wm) * 32 + 8 * q + 4 * h) =
                    v4i{(int)m[4 * q], (int)m[4 * q + 1], (int)m[4 * q + 2], (int)m[4 * q + 3]};
        }
    }
    __syncthreads();
    if (tid < t.vrows) {
        const u32 m0v = __float_as_uint(rm_l[tid]), m1v = __float_as_uint(rm_l[256 + tid]);
        __hip_atomic_fetch_max(e.amax + t.m0 + tid, m0v > m1v ? m0v : m1v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // every row maximum of this tile is released before the arrival (this also drains the next
    // tile's first stages, so its loop starts without a vmcnt wait)
    pf_release_maxima();
    __syncthreads();
    if (tid == 0) pf_arrive(e.arrive + t.mt);
#pragma unroll
    for (int fm = 0; fm < 4; ++fm)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) act[fm][j][r] = from_agpr(act[fm][j][r]);
}

// The pending requant of a workgroup's previous tile (has: one is pending).
struct PfDefer {
    float (&act)[4][2][16];  // its activations
    const GemmArgs& a;
    uint8_t* smem;
    int nt;       // its column tile
    u32 target;   // arrivals that complete a row tile's maxima
    bool has;
    PfTile t;     // its row tile

    // The exchange wait (normally complete long since), 127 / amax of the tile's rows through LDS,
    // then the requant and stores.  A wait that times out marks the tile for the fix-up launch and
    // stores nothing.
    __device__ __forceinline__ void run()
    {
        if (!has) return;
        has = false;
        const int tid = threadIdx.x;
        const EpiArgs& e = a.epi;
        CB_LDS u32* flag = (CB_LDS u32*)((CB_LDS uint8_t*)smem + kPfFlag);
        if (tid == 0) {
            const u32 ok = pf_wait(e, e.arrive + t.mt, target);
            if (!ok) {
                __hip_atomic_fetch_or(e.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(e.redo + t.mt * a.ntiles + nt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            *flag = ok;
        }
        __syncthreads();
        if (__builtin_amdgcn_readfirstlane(*flag) == 0) return;
        CB_LDS float* inv_l = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfInv);
        float am = 0.0f;
        if (tid < t.vrows) am = __uint_as_float(__hip_atomic_load(e.amax + t.m0 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (!(am > kFltMin)) am = kFltMin;
        inv_l[tid] = 127.0f / am;
        if (nt == 0 && tid < t.vrows) e.yq_scale[t.m0 + tid] = am * kInv127;
        __syncthreads();
        // y from column nt * 128 on: rows past the tile's valid rows lie past the resource's end
        // (their offsets are at least vrows * H - nt * 128 while every valid one is below it, as
        // nt * 128 + 128 <= H or the column check below removes the store)
        const int64_t H = e.H;
        const int64_t c0 = (int64_t)nt * 128;
        const __amdgpu_buffer_rsrc_t yr =
            make_rsrc(e.yq + (int64_t)t.m0 * H + c0, (uint32_t)((int64_t)(t.vrows < 256 ? t.vrows : 256) * H - c0));
        const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6), wm = wave >> 1, wn = wave & 1;
        const int c = lane & 31, qi = c & 3, h = lane >> 5;
        uint32_t ybase[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int cl = wn * 64 + j * 32 + (c & ~3);  // column within the tile's 128
            ybase[j] = c0 + cl < H ? (uint32_t)((wm * 32 + 4 * h + qi) * H + cl) : 0x80000000u;
        }
        // lane (h, c) holds rows (2 fm + wm) * 32 + 8 q + 4 h + i of column c: rint16 of
        // act * (127 / amax), a 4 x 4 byte transpose across each lane quad (lane qi ends with row
        // + qi, columns (c & ~3) .. +3), one dword store per 32-column half
        auto quad_bytes = [&](const int fm, const int q, const int j, const v4f& inv4) -> u32 {
            // clamp-and-narrow == saturating rint16; an all-zero row gives 0 * inf = NaN -> 0
            const u32 x = pack4_i8(rint16_h(act[fm][j][4 * q + 0] * inv4[0]), rint16_h(act[fm][j][4 * q + 1] * inv4[1]),
                                   rint16_h(act[fm][j][4 * q + 2] * inv4[2]), rint16_h(act[fm][j][4 * q + 3] * inv4[3]));
            // step 1 swaps 16-bit halves with lane qi ^ 2, step 2 bytes with qi ^ 1
            const u32 pp = (u32)__builtin_amdgcn_update_dpp(0, (int)x, 0x4E, 0xF, 0xF, false);
            const u32 z = (qi & 2) ? __builtin_amdgcn_perm(x, pp, 0x07060302u) : __builtin_amdgcn_perm(pp, x, 0x05040100u);
            const u32 pz = (u32)__builtin_amdgcn_update_dpp(0, (int)z, 0xB1, 0xF, 0xF, false);
            return (qi & 1) ? __builtin_amdgcn_perm(pz, z, 0x03070105u) : __builtin_amdgcn_perm(pz, z, 0x06020400u);
        };
        if ((H & 7) == 0 && ((uintptr_t)e.yq & 7) == 0) {
            // 8-byte stores: slices q and q + 1 transposed, then one swap with lane c ^ 4 (ds_swizzle,
            // lane-uniform): the lane with bit 2 of c clear keeps slice q's row with columns 4..7
            // from lane c + 4, the other slice q + 1's row with columns 0..3 from lane c - 4
            const bool hi4 = (c >> 2) & 1;
            uint32_t ybase8[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int cl = wn * 64 + j * 32 + (c & ~7);
                ybase8[j] = c0 + cl < H ? (uint32_t)((wm * 32 + 4 * h + qi) * H + cl) : 0x80000000u;
            }
#pragma unroll
            for (int fm = 0; fm < 4; ++fm) {
#pragma unroll
                for (int qp = 0; qp < 2; ++qp) {
                    const v4f ia = *(const CB_LDS v4f*)(inv_l + (2 * fm + wm) * 32 + 16 * qp + 4 * h);
                    const v4f ib = *(const CB_LDS v4f*)(inv_l + (2 * fm + wm) * 32 + 16 * qp + 8 + 4 * h);
                    const uint32_t roff = (uint32_t)((64 * fm + 16 * qp + (hi4 ? 8 : 0)) * H);
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const u32 ya = quad_bytes(fm, 2 * qp, j, ia), yb = quad_bytes(fm, 2 * qp + 1, j, ib);
                        const u32 r = (u32)__builtin_amdgcn_ds_swizzle((int)(hi4 ? ya : yb), 0x101F);
                        typedef unsigned int v2u __attribute__((ext_vector_type(2)));
                        const v2u w = hi4 ? v2u{r, yb} : v2u{ya, r};
                        __builtin_amdgcn_raw_buffer_store_b64(w, yr, ybase8[j] + roff, 0, 0);
                    }
                }
            }
            return;
        }
#pragma unroll
        for (int fm = 0; fm < 4; ++fm) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const v4f inv4 = *(const CB_LDS v4f*)(inv_l + (2 * fm + wm) * 32 + 8 * q + 4 * h);
                const uint32_t roff = (uint32_t)((64 * fm + 8 * q) * H);  // rows below slice (0, 0)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    pf_store4(quad_bytes(fm, q, j, inv4), yr, ybase[j] == 0x80000000u ? ybase[j] : ybase[j] + roff,
                              ((uintptr_t)e.yq & 3) != 0);
            }
        }
    }
};

// Persistent GroupedMatmulSwigluQuant prefill kernel.  gridDim.x workgroups, at most one per CU,
// all resident together (the host checks the occupancy).  Exchange group: the row maxima of
// row tile mt are final once its ntl column tiles have counted at arrive[mt].  GATHER: activation rows
// through the row index.
// DEFER: each tile's requant waits until the workgroup's next K loop is done (PfDefer); needs the
// K loop that carries the next tile's prologue (K of at least kPfDeferMinStages stages).
constexpr int kPfDeferMinStages = 4;

template <bool GATHER, bool DEFER>
__global__ __launch_bounds__(256, 1) void gmsq_prefill_kernel(const GemmArgs a)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int ntl = a.ntiles;
    const PfPlace pl = pf_place(ntl, (int)gridDim.x, (int)blockIdx.x);
    CB_LDS int* tab = (CB_LDS int*)((CB_LDS uint8_t*)smem + kPfOrd);
    const PfOrder ord = pf_build_order(a.gt, pl.RT, tab);
    const int rounds = pf_total_rounds(ord);
    const u32 target = (u32)ntl;  // a row tile's column tiles meet at arrive[mt]
    uint32_t a_rd[4][2], b_rd[4];
    pf_read_offsets(wm, wn, lane, a_rd, b_rd);
    const int nk = __builtin_amdgcn_readfirstlane((int)((a.K + PfCfg::BK - 1) / PfCfg::BK));
    PfOffs offs = pf_offsets<GATHER>(a, wave, lane);

    int q = pl.slot;
    if (q >= rounds) return;
    // Round r of a slot gives its workgroup of column position pl.nt the column tile
    // (pl.nt + r) % ntl: every workgroup takes each column tile in turn.  The tiles whose weight
    // lines sit at slow HBM addresses (a fixed maximum read rate: two of the sixteen column tiles
    // of a 4 KB weight row) then fall to a different workgroup every round, and with the requant
    // deferred past the next K loop (DEFER) a round's late tile is absorbed instead of setting
    // every round's pace.
    auto nt_of = [&](int qq) { return (pl.nt + qq / pl.slots) % ntl; };
    // this tile's scales into LDS slot par (the wait for their loads also waits for the prologue)
    auto put_scales = [&](const PfScales& v, int par) {
        CB_LDS float* sl = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfSc + par * kPfScSlot);
        sl[tid] = v.xs;
        sl[256 + tid] = v.cs;
    };
    PfTile cur_t = pf_round_tile(a.gt, tab, ord, pl.RT, q, pl.rt);
    PfSrc cur;
    int par = 0, rb = 0;  // scale slot and ring slot of the current tile
    // the K loop carries the next tile's prologue when K spans at least 4 stages (the prologue's
    // 3.5 stages then all lie in the last 4 iterations)
    const bool pf = nk >= 4;
    if (cur_t.mt >= 0) {
        cur = pf_src<GATHER>(a, cur_t.g, cur_t.m0, cur_t.vrows, nt_of(q), wave, lane);
        pf_prologue<GATHER>(cur, offs, nk, smem, wave);
        put_scales(pf_scales(a, cur_t, nt_of(q)), par);
    }
    bool first = true;
    float act[4][2][16];  // DEFER: the pending tile's activations
    PfDefer def{act, a, smem, 0, target, false, cur_t};
    for (; q < rounds; q += pl.slots) {
        // opaque: the DMA offsets derived from these (every stage of every loop variant) are
        // computed per tile, not hoisted out of the tile loop and spilled
        offs.a0 = opaque(offs.a0);
        offs.b0 = opaque(offs.b0);
        // the next round's tile of this workgroup: its plan and scales are prepared now, and its
        // first stages are fetched by this tile's K loop past K
        const int qn = q + pl.slots;
        const PfTile nxt_t = pf_round_tile(a.gt, tab, ord, pl.RT, qn, pl.rt);
        if (cur_t.mt < 0) {
            // past the last row tile of its kind (no exchange: the counters are per row tile)
            if (DEFER) def.run();
            if (nxt_t.mt >= 0) {
                __syncthreads();
                cur = pf_src<GATHER>(a, nxt_t.g, nxt_t.m0, nxt_t.vrows, nt_of(qn), wave, opaque(lane));
                pf_prologue<GATHER>(cur, offs, nk, smem, wave);
                put_scales(pf_scales(a, nxt_t, nt_of(qn)), par);
                rb = 0;
                first = true;
            }
            cur_t = nxt_t;
            continue;
        }
        PfSrc nxt;
        PfScales nsc;
        if (nxt_t.mt >= 0) {
            nxt = pf_src<GATHER>(a, nxt_t.g, nxt_t.m0, nxt_t.vrows, nt_of(qn), wave, opaque(lane));
            nsc = pf_scales(a, nxt_t, nt_of(qn));
        } else {
            nxt = pf_dead(a);
        }
        v16i acc[4][4];  // defined by the K loop (its first MFMAs start from zero)
        // 32-row blocks with valid rows: wave row wm multiplies fragments fm with 2 fm + wm < nblk
        const int nblk = (cur_t.vrows + 31) / 32;
        const int nv = __builtin_amdgcn_readfirstlane(nblk > wm ? min((nblk - wm + 1) / 2, 4) : 0);
        if (!first && !pf) {
            // K below 4 stages: the previous loop could not carry this tile's prologue
            pf_prologue<GATHER>(cur, offs, nk, smem, wave);
            rb = 0;
            first = true;
        }
        if constexpr (DEFER) {
            // pf holds (nk >= kPfDeferMinStages)
            if (nv >= 4) pf_kloop<4, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 3) pf_kloop<3, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 2) pf_kloop<2, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 1) pf_kloop<1, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else pf_kloop<0, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            def.run();
            pf_publish(a, smem, acc, cur_t, par, act);
            def.has = true;
            def.t = cur_t;
            def.nt = nt_of(q);
        } else if (pf) {
            if (nv >= 4) pf_kloop<4, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 3) pf_kloop<3, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 2) pf_kloop<2, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 1) pf_kloop<1, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else pf_kloop<0, true, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
        } else {
            if (nv >= 4) pf_kloop<4, false, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 3) pf_kloop<3, false, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 2) pf_kloop<2, false, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else if (nv == 1) pf_kloop<1, false, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
            else pf_kloop<0, false, GATHER>(cur, nxt, offs, nk, rb, smem, a_rd, b_rd, acc, wave, first);
        }
        if constexpr (!DEFER) pf_epilogue<false>(a, smem, acc, cur_t, nt_of(q), par, cur_t.mt, target, cur_t.mt * ntl + nt_of(q));
        if (nxt_t.mt >= 0) put_scales(nsc, par ^ 1);
        // every wave is past its LDS reads of this epilogue (and the next scales are written)
        // before the next tile's epilogue
        __syncthreads();
        rb = (rb + nk) & 3;
        par ^= 1;
        if (nxt_t.mt >= 0) cur = nxt;
        first = false;
        cur_t = nxt_t;
    }
    if (DEFER) def.run();
}

// Fix-up launch: recomputes the tiles whose exchange wait timed out (redo[mt * ntl + nt] != 0),
// now that every row maximum is final.  Without a timeout in the main launch (status word 0) every
// workgroup exits at once.
template <bool GATHER>
__global__ __launch_bounds__(256, 1) void gmsq_prefill_fixup_kernel(const GemmArgs a)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(a.epi.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0)
        return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int ntl = a.ntiles;
    const int total = a.gt.total_mtiles * ntl;
    const int nk = __builtin_amdgcn_readfirstlane((int)((a.K + PfCfg::BK - 1) / PfCfg::BK));
    uint32_t a_rd[4][2], b_rd[4];
    pf_read_offsets(wm, wn, lane, a_rd, b_rd);
    for (int t = blockIdx.x; t < total; t += gridDim.x) {
        if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(a.epi.redo + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0)
            continue;
        const int nt = t % ntl;
        const PfTile tl = pf_tile_at(a.gt, t / ntl);
        const PfOffs offs = pf_offsets<GATHER>(a, wave, opaque(lane));
        const PfSrc cur = pf_src<GATHER>(a, tl.g, tl.m0, tl.vrows, nt, wave, opaque(lane));
        __syncthreads();
        pf_prologue<GATHER>(cur, offs, nk, smem, wave);
        {
            const PfScales sc = pf_scales(a, tl, nt);
            CB_LDS float* sl = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfSc);
            sl[tid] = sc.xs;
            sl[256 + tid] = sc.cs;
        }
        v16i acc[4][4];  // defined by the K loop (its first MFMAs start from zero)
        pf_kloop<4, false, GATHER>(cur, cur, offs, nk, 0, smem, a_rd, b_rd, acc, wave, true);
        pf_epilogue<true>(a, smem, acc, tl, nt, 0, 0, 0, t);
        __syncthreads();
    }
}

}  // namespace cb
