// gemm_lds.hpp - the prefill / dense int8 GEMM core: direct-to-LDS loads + transposing LDS reads.
//
// Tile 256 (rows) x 256 (weight columns) x 64 (K), STAGES-deep LDS ring.  Global -> LDS traffic
// uses buffer_load_dwordx4 ... lds (each lane's 16 bytes land at lane-linear LDS addresses, no
// VGPR staging).  Both tiles keep their HBM layout in LDS and are XOR-swizzled at 16-byte
// granularity by choosing which global chunk each lane fetches:
//   A tile [256][64] (K contiguous, 64-byte rows):  position p of row r holds k-chunk p ^ ((r >> 2) & 3)
//   B tile [64][256] (N contiguous, 256-byte rows): position p of row k holds column chunk
//                                                   p ^ ((k & 7) << 1)
// MFMA v_mfma_i32_32x32x32_i8 operands:
//   A: ds_read_b128 of 16 consecutive K bytes of one row.
//   B: two ds_read_b64_tr_b8 per operand.  Within each group of 16 lanes the instruction returns
//      to lane i byte j the byte (i & 7) of the 8 bytes read by lane 2 j + (i >> 3); lane s of a
//      group therefore reads row kb + (s >> 1), columns c0 + 8 (s & 1) .. +8, and lane i receives
//      8 consecutive K values of column c0 + i: the weight is transposed by the LDS read itself.
// The swizzles make every 16-lane phase of those reads touch 16 distinct 16-byte bank groups.
#pragma once

#include <type_traits>

#include "gemm_i8.hpp"

namespace cb {

typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
#define CB_LDS __attribute__((address_space(3)))

// The LDS DMA and the stage barrier are written as inline asm on purpose: when the compiler sees
// buffer_load ... lds it must assume every later LDS read may alias the DMA target and waits for
// vmcnt(0), and a __syncthreads() fence also drains vmcnt - either would serialise the stage
// pipeline.  The waits below are explicit instead: before stage kt is read, each wave waits until
// only the DMAs of later stages are outstanding, then the barrier publishes every wave's stage.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t lds_addr)
{
    asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(rsrc),
                 "s"(lds_addr)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Workgroup barrier after the main loop: every wave's LDS reads and DMAs (including the stages
// issued past the end of K) are drained, so the stage buffers can be reused for epilogue staging.
__device__ __forceinline__ void epi_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vmcnt_barrier()
{
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

template <int WM, int WN, int STAGES, int BK_ = 64>
struct LdsCfg {
    static constexpr int BM = 256, BN = 256, BK = BK_, STAGES_ = STAGES;
    static constexpr int KS = BK / 32;    // 32-deep MFMA steps per stage
    static constexpr int ACH = BK / 16;   // 16-byte chunks per A row
    static_assert(BK == 64 || BK == 128, "stage depth");
    static constexpr int NW = WM * WN, NT = 64 * NW;
    static constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    static constexpr int A_BYTES = BM * BK, B_BYTES = BK * BN, STAGE = A_BYTES + B_BYTES;
    // epilogue staging of the finished tile: 256 rows x 512 bytes (bf16 [256][256] or fp32
    // [256][128]) with a 16-byte row pad that keeps rows 4 apart off the same banks
    static constexpr int EPI_PITCH = 528;
    static constexpr int EPI_BYTES = BM * EPI_PITCH;
    // the tile's per-row activation scales (SwiGLU epilogues), after the ring / staging area
    // and the column scales: one slot of BM + BN floats
    static constexpr int XS_OFF = STAGES * STAGE > EPI_BYTES ? STAGES * STAGE : EPI_BYTES;
    static constexpr int XS_SLOT = (BM + BN) * 4;
    static constexpr int LDS_BYTES = XS_OFF + XS_SLOT;
    // persistent dequant / int32 kernel: the ring, then two scale slots (alternate tiles)
    static constexpr int CONT_XS_OFF = STAGES * STAGE;
    static constexpr int CONT_LDS_BYTES = CONT_XS_OFF + 2 * XS_SLOT;
    static constexpr int A_ISSUE = A_BYTES / 16 / NT;  // DMA instructions per thread per stage
    static constexpr int B_ISSUE = B_BYTES / 16 / NT;
    static constexpr int ISSUE = A_ISSUE + B_ISSUE;
    static_assert(A_ISSUE >= 1 && B_ISSUE >= 1, "tile too small for the workgroup");
    static_assert(FN >= 2 && FN % 2 == 0, "wave tile must hold gate/up pairs");
};

// Global -> LDS DMA plan of one tile: the A and B buffer resources and each lane's stage-independent
// source offsets.  A swizzle key: spreads the 16 rows of a ds_read_b128 phase over all 64 banks
// (BK 64: 4 rows per 256 bytes, key (r >> 2) & 3; BK 128: 2 rows per 256 bytes, key (r >> 1) & 7).
template <int ACH>
__device__ __forceinline__ int a_swizzle(int r) { return ACH == 4 ? ((r >> 2) & 3) : ((r >> 1) & 7); }

template <class C, bool SW>
struct TileDma {
    __amdgpu_buffer_rsrc_t ares, bres;
    uint32_t a_off[C::A_ISSUE], b_off[C::B_ISSUE];
    uint32_t n;  // weight row length
    int nk;

    __device__ __forceinline__ void init(const GemmArgs& a, const int mt, const int nt, const int64_t b, const int wave,
                                         const int lane)
    {
        const int g = group_of_tile(a.gt, mt);
        const int m0 = (g ? a.gt.row_end[g - 1] : 0) + (mt - a.gt.tile_start[g]) * C::BM;
        init_at(a, g, m0, a.gt.row_end[g] - m0, nt, b, wave, lane);
    }

    // The plan of the tile of group g whose rows start at m0 (vrows of them valid).
    __device__ __forceinline__ void init_at(const GemmArgs& a, const int g, const int m0, const int vrows, const int nt,
                                            const int64_t b, const int wave, const int lane)
    {
        constexpr int BM = C::BM, BN = C::BN, NW = C::NW, ACH = C::ACH;
        const int64_t K = a.K, N = a.N;
        // A = rows [m0, r1) of x (with a row index: all of x, rows gathered through the per-lane
        // offsets), B = this group's weight [K, N]
        const bool gather = a.row_index != nullptr;
        ares = gather ? make_rsrc(a.x, (uint32_t)(a.x_rows * K))
                      : make_rsrc(a.x + b * a.x_bstride + (int64_t)m0 * K, (uint32_t)((int64_t)(vrows < BM ? vrows : BM) * K));
        bres = make_rsrc(a.w + b * a.w_bstride + (int64_t)g * a.w_gstride, (uint32_t)(K * N));
        n = (uint32_t)N;
        nk = (int)((K + C::BK - 1) / C::BK);
#pragma unroll
        for (int i = 0; i < C::A_ISSUE; ++i) {
            const int cid = (i * NW + wave) * 64 + lane;  // 16-byte chunk id in the A tile
            const int row = cid / ACH, pos = cid % ACH;
            const int q = pos ^ a_swizzle<ACH>(row);
            // rows past the tile's valid rows (and gathered rows outside x) point past the resource:
            // they read zeros and fetch nothing, so a partial tile moves only its valid rows
            const int srow = row < vrows ? (gather ? src_row(a, m0 + row) : row) : -1;
            a_off[i] = srow >= 0 ? (uint32_t)srow * (uint32_t)K + (uint32_t)(q * 16) : 0x80000000u;
        }
#pragma unroll
        for (int i = 0; i < C::B_ISSUE; ++i) {
            const int cid = (i * NW + wave) * 64 + lane;
            const int row = cid >> 4, pos = cid & 15;
            const int c = pos ^ ((row & 7) << 1);  // logical 16-column chunk
            int64_t col;
            bool ok;
            if constexpr (SW) {
                const int64_t j = (int64_t)nt * (BN / 2) + 16 * (c & 7);
                ok = j < a.epi.H;
                col = c < 8 ? j : a.epi.H + j;
            } else {
                col = (int64_t)nt * BN + 16 * c;
                ok = col < N;
            }
            b_off[i] = (uint32_t)row * (uint32_t)N + (uint32_t)(ok ? col : 0);
        }
    }

    // A plan that fetches nothing (every offset lies outside an empty resource): the stage stream
    // of a persistent workgroup past its last tile.
    __device__ __forceinline__ void set_dead(const GemmArgs& a)
    {
        ares = make_rsrc(a.x, 0u);
        bres = make_rsrc(a.w, 0u);
#pragma unroll
        for (int i = 0; i < C::A_ISSUE; ++i) a_off[i] = 0x80000000u;
#pragma unroll
        for (int i = 0; i < C::B_ISSUE; ++i) b_off[i] = 0x80000000u;
        n = 0;
        nk = 0;
    }

    // DMA chunk I of stage kt (I < A_ISSUE: activation chunk I, else weight chunk I - A_ISSUE) into
    // ring slot `slot`; the same addressing as issue_at.
    template <int I>
    __device__ __forceinline__ void issue_one(const int kt, const int slot, const uint32_t lds_base, const int wave) const
    {
        constexpr int NW = C::NW;
        const uint32_t sa = lds_base + (uint32_t)(slot * C::STAGE);
        if constexpr (I < C::A_ISSUE) {
            dma16(ares, kt < nk ? a_off[I] + (uint32_t)(kt * C::BK) : 0x80000000u,
                  __builtin_amdgcn_readfirstlane(sa + (uint32_t)((I * NW + wave) * 1024)));
        } else {
            constexpr int J = I - C::A_ISSUE;
            dma16(bres, b_off[J] + (uint32_t)(kt * C::BK) * n,
                  __builtin_amdgcn_readfirstlane(sa + C::A_BYTES + (uint32_t)((J * NW + wave) * 1024)));
        }
    }

    // DMAs of stage kt into ring slot kt % STAGES.
    __device__ __forceinline__ void issue(const int kt, const uint32_t lds_base, const int wave) const
    {
        issue_at(kt, kt % C::STAGES_, lds_base, wave);
    }

    // DMAs of stage kt into ring slot `slot`.  Stages past K keep the DMA count (and so every
    // wait) constant but fetch nothing: weight offsets past K*N already lie outside their resource,
    // activation offsets would run into the next rows, so they are moved outside the resource too.
    __device__ __forceinline__ void issue_at(const int kt, const int slot, const uint32_t lds_base,
                                             const int wave) const
    {
        constexpr int NW = C::NW;
        const uint32_t sa = lds_base + (uint32_t)(slot * C::STAGE);
        const uint32_t sb = sa + C::A_BYTES;
        const uint32_t ka = (uint32_t)(kt * C::BK);
        const uint32_t kb = (uint32_t)(kt * C::BK) * n;
        const bool live = kt < nk;
#pragma unroll
        for (int i = 0; i < C::A_ISSUE; ++i)
            dma16(ares, live ? a_off[i] + ka : 0x80000000u,
                  __builtin_amdgcn_readfirstlane(sa + (uint32_t)((i * NW + wave) * 1024)));
#pragma unroll
        for (int i = 0; i < C::B_ISSUE; ++i)
            dma16(bres, b_off[i] + kb, __builtin_amdgcn_readfirstlane(sb + (uint32_t)((i * NW + wave) * 1024)));
    }
};

template <int EPI, int WM, int WN, int STAGES, int BKT>
using TileDmaOf = TileDma<LdsCfg<WM, WN, STAGES, BKT>, false>;

// One 256 x 256 output tile (row tile mt, column tile nt, batch b).  Called once per workgroup by
// lds_gemm_kernel and in a loop by the persistent kernels.
//
// CONT (continuous stage stream, persistent dequant / int32 kernel): the tile's first STAGES stages
// were already issued by the previous tile (or the kernel's prologue) from the plan `cur` into ring
// slots sbase, sbase + 1, ...; the last STAGES iterations of this tile issue the first stages of
// the plan `nxt`.  The epilogue then writes from registers and leaves the LDS ring to those DMAs.
template <int EPI, int WM, int WN, int STAGES, int BKT, bool CONT = false>
__device__ __forceinline__ void lds_gemm_tile(const GemmArgs& a, const int mt, const int nt, const int64_t b,
                                              uint8_t* smem,
                                              const TileDmaOf<EPI, WM, WN, STAGES, BKT>* cur = nullptr,
                                              const TileDmaOf<EPI, WM, WN, STAGES, BKT>* nxt = nullptr,
                                              const int sbase = 0, const int xs_slot = 0)
{
    using C = LdsCfg<WM, WN, STAGES, BKT>;
    constexpr int KS = C::KS, ACH = C::ACH;
    constexpr int BM = C::BM, BN = C::BN, BK = C::BK, TN = C::TN, FM = C::FM,
                  FN = C::FN;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int64_t N = a.N;
    const EpiArgs& e = a.epi;

    const int g = group_of_tile(a.gt, mt);
    const int rs = g ? a.gt.row_end[g - 1] : 0;
    const int r1 = a.gt.row_end[g];
    const int m0 = rs + (mt - a.gt.tile_start[g]) * BM;
    const int vrows = r1 - m0;  // valid rows of this tile (>= 1)

    static_assert(EPI == EPI_DEQUANT || EPI == EPI_I32, "dequant / int32 epilogues only");
    TileDma<C, false> dma;
    if constexpr (CONT) dma = *cur;
    else dma.init(a, mt, nt, b, wave, lane);
    const uint32_t lds_base = (uint32_t)(uintptr_t)(CB_LDS uint8_t*)smem;
    const int nk = dma.nk;
    auto slot_of = [&](int kt) { return CONT ? (sbase + kt) % STAGES : kt % STAGES; };
    auto issue_stage = [&](int kt) {
        if constexpr (CONT) {
            // uniform branch right after a barrier that drained lgkmcnt: nothing for the compiler
            // to wait on at the join
            if (kt < nk) dma.issue_at(kt, slot_of(kt), lds_base, wave);
            else nxt->issue_at(kt - nk, slot_of(kt), lds_base, wave);
        } else {
            dma.issue(kt, lds_base, wave);
        }
    };

    auto tcol = [&](int fn) -> int { return wn * TN + fn * 32; };  // first tile column of fragment fn

    // ---- per-lane LDS read offsets ----------------------------------------------------------
    // A: fragment fm of wave row wm covers tile rows 32 (WM fm + wm) .. +32 (row blocks are
    // interleaved over the WM waves so a partial tile loads them evenly); lane % 32 picks the row,
    // k-chunk q = 2 ks + lane / 32
    uint32_t a_rd[FM][KS];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
        const int r = (WM * fm + wm) * 32 + (lane & 31);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int q = 2 * ks + (lane >> 5);
            a_rd[fm][ks] = (uint32_t)(r * BK + ((q ^ a_swizzle<ACH>(r)) << 4));
        }
    }
    // B: group gq = lane / 16 -> k half (gq >> 1), column half (gq & 1); in-group lane s -> row
    // offset s >> 1, byte half s & 1.  The read of (fn, ks, hf) covers stage row
    // ks * 32 + (gq >> 1) * 16 + hf * 8 + (s >> 1), whose swizzle key (row & 7) = s >> 1 does not
    // depend on ks or hf: one base offset per fragment, the rest are instruction immediates.
    const int gq = lane >> 4, s = lane & 15;
    uint32_t b_rd[FN];
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
        const int cc = (tcol(fn) >> 4) + (gq & 1);
        const int row = (gq >> 1) * 16 + (s >> 1);
        const int pos = cc ^ ((s >> 1) << 1);
        b_rd[fn] = (uint32_t)(C::A_BYTES + row * BN + pos * 16 + (s & 1) * 8);
    }
    auto b_rd_at = [&](int fn, int ks, int hf) -> uint32_t { return b_rd[fn] + (uint32_t)((ks * 32 + hf * 8) * BN); };

    // 32-row fragments of this wave that hold valid rows (wave-uniform); tiles at a group's end run
    // a loop variant without the MFMAs of the empty fragments
    const int nblk = (vrows + 31) / 32;
    const int nvf = __builtin_amdgcn_readfirstlane(nblk > wm ? ((nblk - wm + WM - 1) / WM > FM ? FM : (nblk - wm + WM - 1) / WM) : 0);

    v16i acc[FM][FN];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[fm][fn][r] = 0;

    // Prologue: every LDS buffer gets a stage in flight.  The loop below issues one stage per
    // iteration unconditionally, so the number of DMAs in flight is always the same and every
    // wait is a compile-time constant; stages past the end of K only fetch zeros or unused bytes
    // into buffers that are never read again.
    if constexpr (!CONT) {
#pragma unroll
        for (int st = 0; st < STAGES; ++st) issue_stage(st);
    }
    // Scales of the epilogue, fetched now so the loads hide under the K loop; the epilogue reads
    // them from LDS.  Row scales (the per-token scale, 1 without one): thread tid takes tile row
    // tid % BM.  Column scales (the output scale): thread tid takes tile column tid % BN.  Every
    // thread loads, with no branch around a load: absent operands read through empty buffer
    // resources.
    float xs_pre = 1.0f, cs_pre = 0.0f;
    if constexpr (EPI == EPI_DEQUANT) {
        const int lr0 = tid % BM;
        const __amdgpu_buffer_rsrc_t pres =
            e.has_pt ? make_rsrc(e.pertoken + m0, (uint32_t)((vrows < BM ? vrows : BM) * 4)) : make_rsrc(a.x, 0u);
        const float v = __builtin_bit_cast(
            float, __builtin_amdgcn_raw_buffer_load_b32(pres, (uint32_t)((lr0 < vrows ? lr0 : vrows - 1) * 4), 0, 0));
        xs_pre = e.has_pt ? v : 1.0f;
        // output scale of column cc: fp32 or bf16, per channel or one per group / batch
        const int64_t cc = (int64_t)nt * BN + tid % BN;
        const int64_t si = (int64_t)g * e.scale_gstride + (e.scale_perchan ? (cc < N ? cc : 0) : 0);
        const __amdgpu_buffer_rsrc_t s32 = make_rsrc(e.scale, e.scale_bf16 ? 0u : 0x80000000u);
        const __amdgpu_buffer_rsrc_t s16 = make_rsrc(e.scale, e.scale_bf16 ? 0x80000000u : 0u);
        const float f32 = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s32, (uint32_t)(si * 4), 0, 0));
        const uint16_t b16 = __builtin_amdgcn_raw_buffer_load_b16(s16, (uint32_t)(si * 2), 0, 0);
        cs_pre = e.scale_bf16 ? bf16_to_f32(b16) : f32;
    }
    CB_LDS float* xs_lds =
        (CB_LDS float*)((CB_LDS uint8_t*)smem + (CONT ? C::CONT_XS_OFF + xs_slot * C::XS_SLOT : C::XS_OFF));
    CB_LDS float* cs_lds = xs_lds + BM;
    auto publish_scales = [&]() {
        if (tid < BM) xs_lds[tid] = xs_pre;
        if (tid < BN) cs_lds[tid] = cs_pre;
    };
    if constexpr (CONT && EPI == EPI_DEQUANT) {
        // no barrier of its own in this epilogue: the K loop's barriers publish the slot (the
        // previous tile read the other one)
        publish_scales();
    }

    // Software pipeline per stage kt (fragments of half-stage ks = 0 already in registers):
    //   read ks = 1 fragments | MFMAs on ks = 0 | barrier for stage kt + 1, refill the buffer
    //   of stage kt, read kt + 1 ks = 0 fragments | MFMAs on ks = 1
    // Within each half the reads are interleaved one-for-one with the MFMAs (sched_group_barrier),
    // which keeps at most one fragment set of LDS reads outstanding: the in-order lgkmcnt counter
    // (4 bits) then lets each MFMA wait only for the set it consumes.
    auto kloop = [&](auto nv_const) {
        constexpr int NV = decltype(nv_const)::value;  // fragments that get MFMAs
        constexpr int NVA = NV > 0 ? NV : 1;
        v4i a0[NVA], b0[FN], a1[NVA], b1[FN];
        auto load = [&](int kt, int ks, v4i (&af)[NVA], v4i (&bf)[FN]) {
            if constexpr (NV > 0) {
                const CB_LDS uint8_t* base = (const CB_LDS uint8_t*)smem + slot_of(kt) * C::STAGE;
#pragma unroll
                for (int fm = 0; fm < NV; ++fm) af[fm] = *(const CB_LDS v4i*)(base + a_rd[fm][ks]);
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) {
                    const v2i lo = __builtin_amdgcn_ds_read_tr8_b64_v2i32((CB_LDS v2i*)(base + b_rd_at(fn, ks, 0)));
                    const v2i hi = __builtin_amdgcn_ds_read_tr8_b64_v2i32((CB_LDS v2i*)(base + b_rd_at(fn, ks, 1)));
                    bf[fn] = v4i{lo[0], lo[1], hi[0], hi[1]};
                }
            }
        };
        auto mma = [&](const v4i (&af)[NVA], const v4i (&bf)[FN]) {
            if constexpr (NV > 0) {
#pragma unroll
                for (int fm = 0; fm < NV; ++fm)
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
                        acc[fm][fn] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[fm], bf[fn], acc[fm][fn], 0, 0, 0);
            }
        };
        // one DS read after each MFMA while reads remain, then the remaining MFMAs
        auto interleave = [&]() {
            if constexpr (NV > 0) {
                constexpr int NMFMA = NV * FN, NREAD = NV + 2 * FN;
                constexpr int PAIRS = NMFMA < NREAD ? NMFMA : NREAD;
#pragma unroll
                for (int i = 0; i < PAIRS; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x0008, 1, 0);  // 1 MFMA
                    __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);  // 1 DS read
                }
                if constexpr (NMFMA > PAIRS) __builtin_amdgcn_sched_group_barrier(0x0008, NMFMA - PAIRS, 0);
                if constexpr (NREAD > PAIRS) __builtin_amdgcn_sched_group_barrier(0x0100, NREAD - PAIRS, 0);
            }
        };
        constexpr int LATER = STAGES - 2;  // stages after the awaited one that stay in flight
        wait_vmcnt_barrier<(STAGES - 1) * C::ISSUE>();
        load(0, 0, a0, b0);
        for (int kt = 0; kt < nk; ++kt) {
#pragma unroll
            for (int ks = 0; ks < KS; ks += 2) {
                // step ks (in a0/b0) with step ks + 1 loading, then step ks + 1 with the next
                // stage's first step (or ks + 2) loading
                load(kt, ks + 1, a1, b1);
                mma(a0, b0);
                interleave();
                if (ks + 2 == KS) {
                    wait_vmcnt_barrier<LATER * C::ISSUE>();
                    issue_stage(kt + STAGES);
                    load(kt + 1, 0, a0, b0);
                } else {
                    load(kt, ks + 2, a0, b0);
                }
                mma(a1, b1);
                interleave();
            }
        }
    };
    static_assert(FM <= 4, "loop variants below cover up to 4 fragments");
    if (nvf >= FM) kloop(std::integral_constant<int, FM>());
    else if (FM > 3 && nvf == 3) kloop(std::integral_constant<int, (FM > 3 ? 3 : 0)>());
    else if (FM > 2 && nvf == 2) kloop(std::integral_constant<int, (FM > 2 ? 2 : 0)>());
    else if (FM > 1 && nvf == 1) kloop(std::integral_constant<int, (FM > 1 ? 1 : 0)>());
    else kloop(std::integral_constant<int, 0>());

    bool fvalid[FM];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) fvalid[fm] = fm < nvf;

    // ---- epilogue.  32x32 C layout: lane l holds column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4
    const int lr = (lane >> 5) * 4;
    if constexpr (CONT) {
        // Register-direct epilogue (the LDS ring already receives the next tile's stages).  Stores
        // go through a resource over this tile's valid rows: rows past the group, including whole
        // fragments without valid rows (their accumulators stayed zero), are dropped, so there is
        // no branch whose join would make the compiler wait for the stores issued before it.
        // Column offsets of fragment fn: col0 + 32 fn, outside the resource past N.
        const int64_t col0 = (int64_t)nt * BN + wn * TN + (lane & 31);
        if constexpr (EPI == EPI_I32) {
            const __amdgpu_buffer_rsrc_t ores =
                make_rsrc((int32_t*)e.out + b * e.out_bstride + (int64_t)m0 * N, (uint32_t)((vrows < BM ? vrows : BM) * N * 4));
            uint32_t coff[FN];
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) coff[fn] = col0 + 32 * fn < N ? (uint32_t)(col0 + 32 * fn) * 4u : 0x80000000u;
#pragma unroll
            for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int lrow = (WM * fm + wm) * 32 + (r >> 2) * 8 + lr + (r & 3);
                    const uint32_t roff = (uint32_t)lrow * (uint32_t)N * 4u;
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn)
                        __builtin_amdgcn_raw_buffer_store_b32(acc[fm][fn][r], ores, roff + coff[fn], 0, 0);
                }
            }
        } else {
            // Rows r and r + 1 of a lane pair (l, l ^ 1) are swapped so that each lane stores two
            // adjacent columns of one row as one dword: the even lane row r, columns (c, c + 1),
            // the odd lane row r + 1, columns (c - 1, c).
            const __amdgpu_buffer_rsrc_t ores =
                make_rsrc((uint16_t*)e.out + b * e.out_bstride + (int64_t)m0 * N, (uint32_t)((vrows < BM ? vrows : BM) * N * 2));
            const bool odd = lane & 1;
            ColDeq cd[FN];
            uint32_t coff[FN];
            const bool full_chain = e.has_offset || e.bias_kind != BIAS_NONE;  // uniform
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
                const int64_t cc = col0 + 32 * fn;
                if (full_chain) cd[fn] = col_deq(e, g, b, cc < N ? cc : 0);
                else cd[fn] = ColDeq{cs_lds[wn * TN + fn * 32 + (lane & 31)], 0.0f, 0.0f};
                coff[fn] = cc < N ? (uint32_t)(cc & ~(int64_t)1) * 2u : 0x80000000u;
            }
            // the row scales come from LDS (fetched under the K loop): no global load between the
            // stores, whose wait would drain every store issued before it (vmcnt counts stores too)
            float ptv[FM][16];
#pragma unroll
            for (int fm = 0; fm < FM; ++fm)
#pragma unroll
                for (int r = 0; r < 16; ++r) ptv[fm][r] = xs_lds[(WM * fm + wm) * 32 + (r >> 2) * 8 + lr + (r & 3)];
            auto store = [&](auto simple_const) {
                constexpr bool SIMPLE = decltype(simple_const)::value;
#pragma unroll
                for (int fm = 0; fm < FM; ++fm) {
    #pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        const int lrow = (WM * fm + wm) * 32 + (r >> 2) * 8 + lr + (r & 3);  // rows lrow, lrow + 1
                        const float pt0 = ptv[fm][r], pt1 = ptv[fm][r + 1];
                        const uint32_t roff = (uint32_t)(lrow + (odd ? 1 : 0)) * (uint32_t)N * 2u;
#pragma unroll
                        for (int fn = 0; fn < FN; ++fn) {
                            uint32_t h0, h1;
                            if constexpr (SIMPLE) {
                                h0 = f32_to_bf16_hw(((float)acc[fm][fn][r] * cd[fn].scale) * pt0);
                                h1 = f32_to_bf16_hw(((float)acc[fm][fn][r + 1] * cd[fn].scale) * pt1);
                            } else {
                                const float v0 = apply_deq(e, cd[fn], acc[fm][fn][r], pt0);
                                const float v1 = apply_deq(e, cd[fn], acc[fm][fn][r + 1], pt1);
                                h0 = e.out_bf16 ? f32_to_bf16_hw(v0) : f32_to_f16(v0);
                                h1 = e.out_bf16 ? f32_to_bf16_hw(v1) : f32_to_f16(v1);
                            }
                            const uint32_t p = h0 | (h1 << 16);
                            // partner lane's pair (quad_perm [1, 0, 3, 2])
                            const uint32_t q = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)p, 0xB1, 0xF, 0xF, false);
                            const uint32_t w = odd ? ((q >> 16) | (p & 0xffff0000u)) : ((p & 0xffffu) | (q << 16));
                            __builtin_amdgcn_raw_buffer_store_b32(w, ores, roff + coff[fn], 0, 0);
                        }
                    }
                }
            };
            if (!e.has_offset && e.bias_kind == BIAS_NONE && e.out_bf16)
                store(std::integral_constant<bool, true>());
            else
                store(std::integral_constant<bool, false>());
        }
    } else if constexpr (EPI == EPI_I32) {
        int32_t* ob = (int32_t*)e.out + b * e.out_bstride;
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
            if (!fvalid[fm]) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + (WM * fm + wm) * 32 + (r >> 2) * 8 + lr + (r & 3);
                if (row >= r1) continue;
#pragma unroll
                for (int fn = 0; fn < FN; ++fn) {
                    const int64_t col = (int64_t)nt * BN + wn * TN + fn * 32 + (lane & 31);
                    if (col < N) ob[(int64_t)row * N + col] = acc[fm][fn][r];
                }
            }
        }
    } else {
        // bf16 / fp16 tile [256][256] staged in LDS, then written with 16-byte stores
        const bool full_chain = e.has_offset || e.bias_kind != BIAS_NONE;  // uniform
        ColDeq cd[FN];
        if (full_chain) {
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) {
                const int64_t cc = (int64_t)nt * BN + wn * TN + fn * 32 + (lane & 31);
                cd[fn] = col_deq(e, g, b, cc < N ? cc : 0);
            }
        }
        publish_scales();  // published by the barrier below
        epi_barrier();
        if (!full_chain) {
#pragma unroll
            for (int fn = 0; fn < FN; ++fn) cd[fn] = ColDeq{cs_lds[wn * TN + fn * 32 + (lane & 31)], 0.0f, 0.0f};
        }
        CB_LDS uint8_t* st = (CB_LDS uint8_t*)smem;
        // The flags are uniform: branch once per tile rather than per value, so the common chain
        // (per-channel scale, optional pertoken, no offset or bias, bf16 out: QuantMatmul and the
        // down-projection) runs without the selects of every other variant.  Its arithmetic is
        // apply_deq's for those flags (v * 1.0f when there is no pertoken scale is exact).
        auto stage = [&](auto simple_const) {
            constexpr bool SIMPLE = decltype(simple_const)::value;
#pragma unroll
            for (int fm = 0; fm < FM; ++fm) {
                if (!fvalid[fm]) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int lrow = (WM * fm + wm) * 32 + (r >> 2) * 8 + lr + (r & 3);
                    const float pt = xs_lds[lrow];  // 1 without a per-token scale
#pragma unroll
                    for (int fn = 0; fn < FN; ++fn) {
                        uint16_t h;
                        if constexpr (SIMPLE) {
                            h = f32_to_bf16_hw(((float)acc[fm][fn][r] * cd[fn].scale) * pt);
                        } else {
                            const float v = apply_deq(e, cd[fn], acc[fm][fn][r], pt);
                            h = e.out_bf16 ? f32_to_bf16_hw(v) : f32_to_f16(v);
                        }
                        const int lcol = wn * TN + fn * 32 + (lane & 31);
                        *(CB_LDS uint16_t*)(st + lrow * C::EPI_PITCH + lcol * 2) = h;
                    }
                }
            }
        };
        if (!e.has_offset && e.bias_kind == BIAS_NONE && e.out_bf16)
            stage(std::integral_constant<bool, true>());
        else
            stage(std::integral_constant<bool, false>());
        epi_barrier();
        uint16_t* ob = (uint16_t*)e.out + b * e.out_bstride;
        constexpr int CHUNKS = BM * (BN * 2 / 16);  // 16-byte chunks in the tile
#pragma unroll
        for (int i = 0; i < CHUNKS / C::NT; ++i) {
            const int id = tid + i * C::NT;
            const int lrow = id / (BN * 2 / 16), ch = id % (BN * 2 / 16);
            const int row = m0 + lrow;
            const int64_t col = (int64_t)nt * BN + ch * 8;
            if (row < r1 && col < N)
                *reinterpret_cast<v4i*>(ob + (int64_t)row * N + col) =
                    *(const CB_LDS v4i*)(st + lrow * C::EPI_PITCH + ch * 16);
        }
    }
}

// Tile pid of the non-persistent launch order: GROUP_M row tiles x all column tiles per group of
// pids, so the workgroups resident together share GROUP_M activation slabs and their weights.
__device__ __forceinline__ void tile_of_pid(const GemmArgs& a, const int pid, int& mt, int& nt)
{
    constexpr int GROUP_M = 4;
    const int T_m = a.gt.total_mtiles, T_n = a.ntiles;
    const int per_group = GROUP_M * T_n;
    const int gid = pid / per_group;
    const int first_m = gid * GROUP_M;
    const int gsz = (T_m - first_m) < GROUP_M ? (T_m - first_m) : GROUP_M;
    mt = first_m + (pid % per_group) % gsz;
    nt = (pid % per_group) / gsz;
}

// Non-persistent launch: one tile per workgroup.
template <int EPI, int WM, int WN, int STAGES, int BKT>
__global__ __launch_bounds__(64 * WM * WN, 1) void lds_gemm_kernel(const GemmArgs a)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    // ---- tile selection (GROUP_M swizzle) ---------------------------------------------------
    // Measured on the prefill and dense shapes: the plain dispatch order (workgroups round-robin
    // over the XCDs) is as good as or better than an XCD-contiguous remap of the tile order.
    const int pid = blockIdx.x;
    int mt, nt;
    tile_of_pid(a, pid, mt, nt);
    lds_gemm_tile<EPI, WM, WN, STAGES, BKT>(a, mt, nt, blockIdx.y, smem);
}

// Persistent dequant / int32 GEMM (batch 1): gridDim.x workgroups, one per CU, walk the tiles
// pid = blockIdx.x, blockIdx.x + gridDim.x, ... of the non-persistent order.  One continuous stage
// stream per workgroup: a tile's last STAGES iterations DMA the next tile's first stages, so no tile
// starts with an empty ring, and the register-direct epilogue overlaps those DMAs.
template <int EPI, int WM, int WN, int STAGES, int BKT>
__global__ __launch_bounds__(64 * WM * WN, 1) void lds_gemm_persistent_kernel(const GemmArgs a)
{
    extern __shared__ __attribute__((aligned(1024))) uint8_t smem[];
    const int total = a.gt.total_mtiles * a.ntiles;
    int pid = blockIdx.x;
    if (pid >= total) return;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t lds_base = (uint32_t)(uintptr_t)(CB_LDS uint8_t*)smem;
    TileDmaOf<EPI, WM, WN, STAGES, BKT> cur, nxt;
    int mt, nt;
    tile_of_pid(a, pid, mt, nt);
    cur.init(a, mt, nt, 0, wave, lane);
#pragma unroll
    for (int st = 0; st < STAGES; ++st) cur.issue_at(st, st, lds_base, wave);
    int sbase = 0, xs_slot = 0;
    for (;;) {
        const int pn = pid + (int)gridDim.x;
        int mt2 = 0, nt2 = 0;
        if (pn < total) {
            tile_of_pid(a, pn, mt2, nt2);
            nxt.init(a, mt2, nt2, 0, wave, lane);
        } else {
            nxt.set_dead(a);
        }
        lds_gemm_tile<EPI, WM, WN, STAGES, BKT, true>(a, mt, nt, 0, smem, &cur, &nxt, sbase, xs_slot);
        if (pn >= total) break;
        xs_slot ^= 1;
        sbase = (sbase + cur.nk) % STAGES;
        cur = nxt;
        pid = pn;
        mt = mt2;
        nt = nt2;
    }
    // the dead stages issued by the last tile fetch nothing; drain them before the wave ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

}  // namespace cb
