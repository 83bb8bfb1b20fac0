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
// so 2.5 stages (80 KB) are in flight while one is multiplied.  Stages past K fetch nothing.
//
// Epilogue, per tile:
//   1. wait for every DMA (the dead ones past K), barrier: the ring is free;
//   2. issue the next tile's first 3.5 stages and fetch its scales, so their latency hides under
//      steps 3-6;
//   3. SwiGLU from the accumulators (the reference's operation order), |act| row maxima reduced
//      across lanes (DPP) and across the two waves sharing rows (LDS), one device-scope atomicMax
//      per (row, tile);
//   4. arrival count for the round's exchange group, then a bounded wait until every column tile
//      of the group's row tiles has published;
//   5. per-row 127 / amax through LDS, rint16 in registers, a 4 x 4 byte transpose across each
//      lane quad, and dword stores of int8 y (four consecutive columns per lane).
// A column tile whose wait times out marks itself in the workspace and stores nothing; the fix-up
// launch that always follows recomputes exactly those tiles with the final row maxima, so the
// output is right whatever the residency of the grid (it exits at once when nothing is marked).
#pragma once

#include "gemm_lds.hpp"

namespace cb {


using PfCfg = LdsCfg<2, 2, 4, 64>;
using PfDma = TileDma<PfCfg, true>;

// LDS map (bytes): the ring, then per-row activation scales [256], per-column weight scales
// [256] (128 gate then 128 up), row maxima of the two column-half waves [2][256], 127 / amax [256],
// the round-order table.
constexpr int kPfRing = PfCfg::STAGES_ * PfCfg::STAGE;
constexpr int kPfXs = kPfRing, kPfCs = kPfXs + 1024, kPfRm = kPfCs + 1024, kPfInv = kPfRm + 2048;
constexpr int kPfOrd = kPfInv + 1024;
constexpr int kPfLds = kPfOrd + 3 * 4 * (CB_MAX_EXPERTS + 1);
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
        // Workgroup b is dispatched to XCD b % 8.  Slot s = the XCD pair (2s, 2s + 1); each XCD
        // holds the slot's 4 row tiles x 8 column tiles, so the workgroups sharing an activation
        // slab or a weight slab share one L2.
        const int x = b & 7, j = b >> 3;
        p.slot = x >> 1;
        p.rt = j >> 3;
        p.nt = (x & 1) * 8 + (j & 7);
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
// Ring slot of stage kt: kt % 4 (every tile starts its stage count at slot 0).
template <int NV>
__device__ __forceinline__ void pf_kloop(const PfDma& dma, uint8_t* smem, const uint32_t (&a_rd)[4][2],
                                         const uint32_t (&b_rd)[4], v16i (&acc)[4][4], const int wave,
                                         const bool first)
{
    using C = PfCfg;
    constexpr int NVA = NV > 0 ? NV : 1;
    const uint32_t lds_base = (uint32_t)(uintptr_t)(CB_LDS uint8_t*)smem;
    const CB_LDS uint8_t* sm = (const CB_LDS uint8_t*)smem;
    const int nk = __builtin_amdgcn_readfirstlane(dma.nk);
    v4i a0[NVA], a1[NVA], b0[4], b1[4];
    auto rdb = [&](int kt, int ks, int fn, v4i (&bf)[4]) {
        const CB_LDS uint8_t* base = sm + (kt & 3) * C::STAGE + C::A_BYTES;
        const uint32_t o = b_rd[fn] + (uint32_t)(ks * 32 * C::BN);
        const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((CB_LDS v2i*)(base + o));
        const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((CB_LDS v2i*)(base + o + 8 * C::BN));
        bf[fn] = v4i{lo[0], lo[1], hi[0], hi[1]};
    };
    auto rda = [&](int kt, int ks, int fm, v4i (&af)[NVA]) {
        if (fm < NV) af[fm < NVA ? fm : 0] = *(const CB_LDS v4i*)(sm + (kt & 3) * C::STAGE + a_rd[fm][ks]);
    };
    auto mrow = [&](int fm, const v4i (&af)[NVA], const v4i (&bf)[4]) {
        if (fm < NV) {
#pragma unroll
            for (int fn = 0; fn < 4; ++fn)
                acc[fm][fn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[fm < NVA ? fm : 0], bf[fn], acc[fm][fn], 0, 0, 0);
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
    // drained by its predecessor's epilogue (every VMEM result waited for), so only the barrier
    if (first) wait_vmcnt_barrier<2 * C::ISSUE + C::A_ISSUE>();
    else wait_vmcnt_barrier<63>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0) in the compiler's own accounting
    if constexpr (NV > 0) {
#pragma unroll
        for (int c = 0; c < 4; ++c) rdb(0, 0, c, b0);
#pragma unroll
        for (int c = 0; c < 4; ++c) rda(0, 0, c, a0);
    }
    for (int kt = 0; kt < nk; ++kt) {
        // half 1: MFMAs of step 0 (a0/b0), reads of step 1, the B chunks of stage kt + 3
        const int s3 = (kt + 3) & 3;
        dma.template issue_one<4>(kt + 3, s3, lds_base, wave);
        if constexpr (NV > 0) { rdb(kt, 1, 0, b1); rdb(kt, 1, 1, b1); }
        mrow(0, a0, b0);
        fence();
        dma.template issue_one<5>(kt + 3, s3, lds_base, wave);
        if constexpr (NV > 0) { rdb(kt, 1, 2, b1); rdb(kt, 1, 3, b1); }
        mrow(1, a0, b0);
        fence();
        dma.template issue_one<6>(kt + 3, s3, lds_base, wave);
        rda(kt, 1, 0, a1);
        rda(kt, 1, 1, a1);
        mrow(2, a0, b0);
        fence();
        dma.template issue_one<7>(kt + 3, s3, lds_base, wave);
        rda(kt, 1, 2, a1);
        rda(kt, 1, 3, a1);
        mrow(3, a0, b0);
        fence();
        // stage kt + 1 landed (outstanding: stage kt + 2 and kt + 3), stage kt fully read
        wait_vmcnt_barrier<2 * C::ISSUE>();
        // half 2: MFMAs of step 1 (a1/b1), reads of stage kt + 1 step 0, the A chunks of stage
        // kt + 4 into the slot stage kt just left
        const int s4 = kt & 3;
        dma.template issue_one<0>(kt + 4, s4, lds_base, wave);
        if constexpr (NV > 0) { rdb(kt + 1, 0, 0, b0); rdb(kt + 1, 0, 1, b0); }
        mrow(0, a1, b1);
        fence();
        dma.template issue_one<1>(kt + 4, s4, lds_base, wave);
        if constexpr (NV > 0) { rdb(kt + 1, 0, 2, b0); rdb(kt + 1, 0, 3, b0); }
        mrow(1, a1, b1);
        fence();
        dma.template issue_one<2>(kt + 4, s4, lds_base, wave);
        rda(kt + 1, 0, 0, a0);
        rda(kt + 1, 0, 1, a0);
        mrow(2, a1, b1);
        fence();
        dma.template issue_one<3>(kt + 4, s4, lds_base, wave);
        rda(kt + 1, 0, 2, a0);
        rda(kt + 1, 0, 3, a0);
        mrow(3, a1, b1);
        fence();
    }
}

// Prologue of a tile: stages 0-2 and the A chunks of stage 3 (the loop issues the rest).
__device__ __forceinline__ void pf_prologue(const PfDma& dma, uint8_t* smem, const int wave)
{
    const uint32_t lds_base = (uint32_t)(uintptr_t)(CB_LDS uint8_t*)smem;
#pragma unroll
    for (int st = 0; st < 3; ++st) dma.issue_at(st, st, lds_base, wave);
    dma.template issue_one<0>(3, 3, lds_base, wave);
    dma.template issue_one<1>(3, 3, lds_base, wave);
    dma.template issue_one<2>(3, 3, lds_base, wave);
    dma.template issue_one<3>(3, 3, lds_base, wave);
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
// covers tile rows (2 fm + wm) * 32 + lane % 32, k chunk 2 ks + lane / 32.  B: see TileDma.
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
// no NaN canonicalisation, so each step is one v_max_u32 with a DPP source).  mov_dpp leaves the
// lanes it does not write undefined.
template <int CTRL, int ROWS>
__device__ __forceinline__ u32 umax_dpp(u32 v)
{
    const u32 o = (u32)__builtin_amdgcn_mov_dpp((int)v, CTRL, ROWS, 0xF, false);
    return v > o ? v : o;
}

// rint16 of four values packed into the four bytes of a dword: fp16 rounding (v_cvt_f16_f32),
// fp16 round-half-even, fp16 -> int16 (NaN -> 0, +-inf saturate), then a clamp to [-128, 127]:
// the same steps as rint16 in one fewer pass through fp32.
__device__ __forceinline__ int rint16_h(float v)
{
    // opaque: v is the rounded fp32 product, not folded into a mixed-precision fma with one rounding
    const _Float16 r = __builtin_elementwise_roundeven((_Float16)opaque(v));
    int i;
    asm("v_cvt_i16_f16 %0, %1" : "=v"(i) : "v"(r));
    const short s = (short)i;
    return s < -128 ? -128 : (s > 127 ? 127 : s);
}

// One persistent GMSQ tile after its K loop: everything from the SwiGLU to the int8 stores.
// Returns false when the exchange wait timed out (the tile stored nothing and is marked for the
// fix-up launch).
template <bool FIXUP>
__device__ __forceinline__ void pf_epilogue(const GemmArgs& a, uint8_t* smem, v16i (&acc)[4][4], const PfTile& t,
                                            const int nt, const PfScales& sc, const int arr_idx,
                                            const u32 arr_target, const int tile_id, const PfDma& nxt,
                                            const bool has_nxt)
{
    // opaque: the per-tile address math is recomputed here rather than hoisted out of the tile loop
    // (and spilled across the K loop)
    const int tid = opaque((int)threadIdx.x), lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const EpiArgs& e = a.epi;
    const int64_t H = e.H;
    const int m0 = t.m0, vrows = t.vrows;
    CB_LDS float* xs_l = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfXs);
    CB_LDS float* cs_l = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfCs);
    CB_LDS float* rm_l = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfRm);
    CB_LDS float* inv_l = (CB_LDS float*)((CB_LDS uint8_t*)smem + kPfInv);

    // 1. every DMA of this tile (the dead ones past K included) has landed and every wave has
    //    finished its ring reads; the scales of this tile go to LDS
    xs_l[tid] = sc.xs;
    cs_l[tid] = sc.cs;
    epi_barrier();
    // 2. the next tile's prologue (its plan and scales were prepared before this tile's K loop)
    if (!FIXUP && has_nxt) pf_prologue(nxt, smem, wave);

    // 3. SwiGLU.  Lane (h = lane / 32, c = lane % 32) of fragment (fm, fn) holds rows
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
        // 4. exchange: every row maximum of this tile has completed before the arrival count
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (tid == 0) {
            __hip_atomic_fetch_add(e.arrive + arr_idx, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            int spins = 0;
            u32 ok = 1;
            while (__hip_atomic_load(e.arrive + arr_idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < arr_target) {
                __builtin_amdgcn_s_sleep(8);
                if (++spins > e.spin_limit) {
                    ok = 0;
                    break;
                }
            }
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

    // 5. final row maxima -> 127 / amax through LDS; the nt = 0 tile writes y_scale
    {
        float am = 0.0f;
        if (tid < vrows) am = __uint_as_float(__hip_atomic_load(e.amax + m0 + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        if (!(am > kFltMin)) am = kFltMin;
        inv_l[tid] = 127.0f / am;
        if (nt == 0 && tid < vrows) e.yq_scale[m0 + tid] = am * kInv127;
        // every VMEM result (the next tile's prologue included) is in before the stores below, so
        // the next tile's loop starts without a vmcnt wait
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
                __builtin_amdgcn_raw_buffer_store_b32((int)y, yr, off, 0, 0);
            }
        }
    }
}

// Persistent GroupedMatmulSwigluQuant prefill kernel.  gridDim.x workgroups, at most one per CU,
// all resident together (the host checks the occupancy).  Exchange group q = round q of slot s:
// its RT row tiles x ntl column tiles meet at arrive[q] once per round.
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
    const u32 target = (u32)(pl.RT * ntl);
    uint32_t a_rd[4][2], b_rd[4];
    pf_read_offsets(wm, wn, lane, a_rd, b_rd);

    int q = pl.slot;
    if (q >= rounds) return;
    PfTile cur_t = pf_round_tile(a.gt, tab, ord, pl.RT, q, pl.rt);
    PfDma cur;
    PfScales sc;
    if (cur_t.mt >= 0) {
        cur.init_at(a, cur_t.g, cur_t.m0, cur_t.vrows, pl.nt, 0, wave, lane);
        pf_prologue(cur, smem, wave);
        sc = pf_scales(a, cur_t, pl.nt);
    }
    bool first = true;
    for (; q < rounds; q += pl.slots) {
        // the next round's tile of this workgroup: its plan and scales are prepared now, its
        // prologue is issued by this tile's epilogue
        const int qn = q + pl.slots;
        const PfTile nxt_t = pf_round_tile(a.gt, tab, ord, pl.RT, qn, pl.rt);
        if (cur_t.mt < 0) {
            // past the last row tile of its kind: still take part in the round's exchange
            if (tid == 0) __hip_atomic_fetch_add(a.epi.arrive + q, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (nxt_t.mt >= 0) {
                __syncthreads();
                cur.init_at(a, nxt_t.g, nxt_t.m0, nxt_t.vrows, pl.nt, 0, wave, opaque(lane));
                pf_prologue(cur, smem, wave);
                sc = pf_scales(a, nxt_t, pl.nt);
                first = true;
            }
            cur_t = nxt_t;
            continue;
        }
        PfDma nxt;
        PfScales nsc;
        if (nxt_t.mt >= 0) {
            nxt.init_at(a, nxt_t.g, nxt_t.m0, nxt_t.vrows, pl.nt, 0, wave, opaque(lane));
            nsc = pf_scales(a, nxt_t, pl.nt);
        }
        v16i acc[4][4];
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
            for (int fn = 0; fn < 4; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0;
        // 32-row blocks with valid rows: wave row wm multiplies fragments fm with 2 fm + wm < nblk
        const int nblk = (cur_t.vrows + 31) / 32;
        const int nv = __builtin_amdgcn_readfirstlane(nblk > wm ? min((nblk - wm + 1) / 2, 4) : 0);
        if (nv >= 4) pf_kloop<4>(cur, smem, a_rd, b_rd, acc, wave, first);
        else if (nv == 3) pf_kloop<3>(cur, smem, a_rd, b_rd, acc, wave, first);
        else if (nv == 2) pf_kloop<2>(cur, smem, a_rd, b_rd, acc, wave, first);
        else if (nv == 1) pf_kloop<1>(cur, smem, a_rd, b_rd, acc, wave, first);
        else pf_kloop<0>(cur, smem, a_rd, b_rd, acc, wave, first);
        pf_epilogue<false>(a, smem, acc, cur_t, pl.nt, sc, q, target, cur_t.mt * ntl + pl.nt, nxt, nxt_t.mt >= 0);
        // every wave is past its LDS reads of this epilogue before the next tile writes scales
        __syncthreads();
        if (nxt_t.mt >= 0) {
            cur = nxt;
            sc = nsc;
        }
        first = false;
        cur_t = nxt_t;
    }
}

// Fix-up launch: recomputes the tiles whose exchange wait timed out (redo[mt * ntl + nt] != 0),
// now that every row maximum is final.  With nothing marked every workgroup exits after scanning.
__global__ __launch_bounds__(256, 1) void gmsq_prefill_fixup_kernel(const GemmArgs a)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;
    const int ntl = a.ntiles;
    const int total = a.gt.total_mtiles * ntl;
    uint32_t a_rd[4][2], b_rd[4];
    pf_read_offsets(wm, wn, lane, a_rd, b_rd);
    for (int t = blockIdx.x; t < total; t += gridDim.x) {
        if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(a.epi.redo + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0)
            continue;
        const int nt = t % ntl;
        const PfTile tl = pf_tile_at(a.gt, t / ntl);
        PfDma cur;
        cur.init_at(a, tl.g, tl.m0, tl.vrows, nt, 0, wave, opaque(lane));
        __syncthreads();
        pf_prologue(cur, smem, wave);
        const PfScales sc = pf_scales(a, tl, nt);
        v16i acc[4][4];
#pragma unroll
        for (int fm = 0; fm < 4; ++fm)
#pragma unroll
            for (int fn = 0; fn < 4; ++fn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0;
        pf_kloop<4>(cur, smem, a_rd, b_rd, acc, wave, true);
        pf_epilogue<true>(a, smem, acc, tl, nt, sc, 0, 0, t, cur, false);
        __syncthreads();
    }
}

}  // namespace cb
