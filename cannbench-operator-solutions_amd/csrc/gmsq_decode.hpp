// gmsq_decode.hpp - GroupedMatmulSwigluQuant for decode-shaped groups (at most 32 rows per expert):
// weight streaming, SwiGLU and the per-token requant in one launch.
//
// Reference being replaced: launch_gmsq_cube + launch_gmsq_vec (gmsq_cube_kernel.cpp:48-130,
// gmsq_vec_kernel.cpp:58-270), which round-trip the int32 product through HBM.  Here each
// workgroup = (expert g, 128 act columns) streams its 7168 x 256 weight block once (the skinny core
// of gemm_i8.hpp: 4 waves split K, 16 x 16 in-register byte transposes, v_mfma_i32_16x16x64_i8, an
// exact int32 reduction through LDS), keeps the activation of its (at most 2 x 16) rows on chip
// and publishes one |act| maximum per (row, tile).  Each tile quantises its own slice once the
// ntiles maxima of its rows are all published, so neither the int32 product nor the fp32
// activation leaves the chip.
//
// The wait is bounded, and a tile that gives up marks itself for the fix-up launch (as in the
// prefill kernel), which recomputes it once every maximum is final.
#pragma once

#include "gemm_i8.hpp"

namespace cb {

// The product, SwiGLU and row maxima of one (expert g, 128-act-column) tile.  Lane (q, c), c < 8,
// ends with act[rb][j] = act of row r0 + 16 rb + 4 q + wave, act column 128 ct + 16 c + j, and
// rmax[rb] = the row's maximum |act| over the tile (in every lane of the 16-lane group); lanes
// c >= 8 hold the up partners during the product and zeros after.
__device__ __forceinline__ void decode_tile_act(const GemmArgs& a, const int g, const int ct, const int r0, const int r1,
                                                int (&red)[3][4][16][64], float (&act)[2][16], u32 (&rmax)[2])
{
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4, c = lane & 15;
    const int64_t K = a.K, N = a.N;
    const EpiArgs& e = a.epi;
    const int64_t H = e.H;
    // lanes c < 8: gate columns ocol .. ocol + 15; lanes c >= 8 their up partners (8 lanes away)
    const int64_t ocol = (int64_t)ct * 128 + 16 * (c & 7);
    const bool colok = ocol < H;
    const int64_t col = (c < 8) ? ocol : H + ocol;
    const __amdgpu_buffer_rsrc_t wres = make_rsrc(a.w + (int64_t)g * a.w_gstride, (uint32_t)(K * N));
    const uint32_t lane_off = (uint32_t)(colok ? col : 0) + (uint32_t)(q * 16) * (uint32_t)N;
    const int nch = (int)((K + 63) >> 6);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        rmax[rb] = 0u;
#pragma unroll
        for (int j = 0; j < 16; ++j) act[rb][j] = 0.0f;
        const int mb = r0 + 16 * rb;
        if (mb >= r1) continue;  // uniform
        v4i acc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = v4i{0, 0, 0, 0};
        const SkinnyRow xres = skinny_row(a, 0, mb, r1, c);
        // wave w multiplies chunks w, w + 4, ...; two chunks in flight per wave (register double
        // buffering): the load of chunk kc + 8 goes out as soon as chunk kc is multiplied.  Chunks
        // past K read zeros through both resources (their MFMAs add nothing), so the loop needs no
        // branch around a load.
        uint4 R0[16], R1[16];
        v4i A0, A1;
        skinny_load_chunk(xres, wres, lane_off, (uint32_t)N, q, wave, R0, A0);
        skinny_load_chunk(xres, wres, lane_off, (uint32_t)N, q, wave + 4, R1, A1);
        for (int kc = wave; kc < nch; kc += 8) {
            skinny_mma_chunk(R0, A0, acc);
            skinny_load_chunk(xres, wres, lane_off, (uint32_t)N, q, kc + 8, R0, A0);
            skinny_mma_chunk(R1, A1, acc);
            skinny_load_chunk(xres, wres, lane_off, (uint32_t)N, q, kc + 12, R1, A1);
        }
        // exact cross-wave K reduction: wave w keeps accumulator row w
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
        const int row = mb + 4 * q + wave;
        int u[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) u[j] = __shfl_xor(s[j], 8, 64);
        float m = 0.0f;
        if (c < 8 && row < r1 && colok) {
            const float xs = src_x_scale(a, row);
            const float* wsg = e.w_scale + (int64_t)g * N + opaque(ocol);
            const float* wsu = wsg + H;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                act[rb][j] = swiglu((float)s[j], (float)u[j], xs, wsg[j], wsu[j]);
                m = fmaxf(m, fabsf(act[rb][j]));
            }
        }
        m = fmaxf(m, __shfl_xor(m, 1, 64));
        m = fmaxf(m, __shfl_xor(m, 2, 64));
        m = fmaxf(m, __shfl_xor(m, 4, 64));
        rmax[rb] = __float_as_uint(m);
    }
}

// Row maxima exchange through self-validating slots: tile (g, ct) stores, for each of its rows r,
// slot[r * ntiles + ct] = |act| maximum bits | 0x80000000 (the bit marks the slot as written; the
// workspace starts zeroed).  A row's final maximum is the maximum over its ntiles slots once every
// slot carries the mark, so no separate arrival count (and no wait for the stores) is needed.
__device__ __forceinline__ void decode_publish(const GemmArgs& a, const int ct, const int r0, const int r1,
                                               const u32 (&rmax)[2])
{
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4, c = lane & 15;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int row = r0 + 16 * rb + 4 * q + wave;
        if (c == 0 && row < r1)
            __hip_atomic_store(a.epi.amax + (int64_t)row * a.ntiles + ct, rmax[rb] | 0x80000000u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The final row maxima of this lane's rows (every lane of a 16-lane group gets its row's value),
// polling until all ntiles slots are marked, at most spin_limit times.  Returns false on timeout.
__device__ __forceinline__ bool decode_gather(const GemmArgs& a, const int r0, const int r1, float (&am)[2])
{
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4, c = lane & 15;
    const int ntl = a.ntiles;
    for (int spins = 0;; ++spins) {
        bool all = true;
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const int row = r0 + 16 * rb + 4 * q + wave;
            u32 m = 0u, ok = 1u;
            if (r0 + 16 * rb < r1 && row < r1) {
                for (int j = c; j < ntl; j += 16) {
                    const u32 v = __hip_atomic_load(a.epi.amax + (int64_t)row * ntl + j, __ATOMIC_RELAXED,
                                                    __HIP_MEMORY_SCOPE_AGENT);
                    ok &= v >> 31;
                    const u32 mv = v & 0x7fffffffu;
                    m = mv > m ? mv : m;
                }
            }
#pragma unroll
            for (int o = 1; o < 16; o <<= 1) {
                const u32 m2 = (u32)__shfl_xor((int)m, o, 64), ok2 = (u32)__shfl_xor((int)ok, o, 64);
                m = m2 > m ? m2 : m;
                ok &= ok2;
            }
            am[rb] = __uint_as_float(m);
            all = all && ok;
        }
        if (__builtin_amdgcn_ballot_w64(!all) == 0) return true;  // all 64 lanes' rows are final
        // give up after spin_limit polls, or once any wait of the call has given up (the status
        // word: the rest of the call then leaves its tiles to the fix-up launch at once)
        if (spins >= a.epi.spin_limit ||
            ((spins & 255) == 255 && (__hip_atomic_load(a.epi.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 1u)))
            return false;
        __builtin_amdgcn_s_sleep(4);
    }
}

// y = rint16(act * 127 / amax) with amax floored at FLT_MIN (an all-zero row gives 0 * inf = NaN
// -> 0), 16 bytes per lane; column tile 0 writes y_scale.
__device__ __forceinline__ void decode_tile_quant(const GemmArgs& a, const int ct, const int r0, const int r1,
                                                  const float (&act)[2][16], const float (&amax)[2])
{
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4, c = lane & 15;
    const EpiArgs& e = a.epi;
    const int64_t H = e.H;
    const int64_t ocol = (int64_t)ct * 128 + 16 * (c & 7);
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int row = r0 + 16 * rb + 4 * q + wave;
        if (row < r1) {
            float am = amax[rb];
            if (!(am > kFltMin)) am = kFltMin;
            if (c < 8 && ocol < H) {
                const float inv = 127.0f / am;
                v4i w;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    w[k] = (int)pack4_i8(rint16(act[rb][4 * k] * inv), rint16(act[rb][4 * k + 1] * inv),
                                         rint16(act[rb][4 * k + 2] * inv), rint16(act[rb][4 * k + 3] * inv));
                int8_t* yp = e.yq + (int64_t)row * H + ocol;
                // H % 16 == 0 and ocol % 16 == 0: the address is aligned as y itself (a uniform choice)
                const uintptr_t al = (uintptr_t)e.yq & 15;
                if (al == 0) {
                    *reinterpret_cast<v4i*>(yp) = w;
                } else if ((al & 3) == 0) {
#pragma unroll
                    for (int k = 0; k < 4; ++k) reinterpret_cast<int*>(yp)[k] = w[k];
                } else {
#pragma unroll
                    for (int k = 0; k < 16; ++k) yp[k] = (int8_t)(w[k >> 2] >> (8 * (k & 3)));
                }
            }
            if (ct == 0 && c == 0) e.yq_scale[row] = am * kInv127;
        }
    }
}

// Requant of a finished tile once its rows' maxima are final; a wave that gives up marks the tile
// for the fix-up launch (which redoes the whole tile) and stores nothing.  no_wait: the tile is
// left to the fix-up launch without waiting (status bit 1 instead of the timeout bit 0, so the
// other waits of the call still wait).
__device__ __forceinline__ void decode_finish(const GemmArgs& a, const int g, const int ct, const int r0, const int r1,
                                              const float (&act)[2][16], const bool no_wait = false)
{
    float am[2];
    // a negative poll limit (test hook) gives up at once
    if (!no_wait && a.epi.spin_limit >= 0 && decode_gather(a, r0, r1, am)) {
        decode_tile_quant(a, ct, r0, r1, act, am);
    } else if ((threadIdx.x & 63) == 0) {
        __hip_atomic_fetch_or(a.epi.status, no_wait ? 2u : 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.epi.redo + g * a.ntiles + ct, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Persistent decode kernel with dynamic tile order.  The tiles (expert g, 128-act-column tile ct)
// are numbered in expert order, t = g * ntiles + ct, and the workgroups draw them with one atomic
// ticket, so a faster CU simply takes more tiles.  (Measured: one list in expert order beats 8
// per-XCD lists, each holding a quarter of the experts and half of the columns.)  An expert's
// column tiles are drawn together, so they finish together: each tile publishes its row maxima
// into the self-validating slots as soon as its product is done, and its requant is deferred until
// the workgroup's next tile is done, by which time the expert's other column tiles have normally
// published; the deferred activations wait in LDS.
//
// Progress.  The next ticket is drawn when a tile starts (its latency hides under the tile), so
// while a workgroup waits for its deferred tile P, it holds one drawn ticket D it has not started.
// Tickets are in expert order and a workgroup's D comes after its P, so a workgroup that waits on
// expert g depends only on workgroups whose unstarted D lies in expert g, and those wait on
// experts no later than g.  Along a chain of waits the experts never increase, so a cycle needs a
// workgroup whose own D lies in its own P's expert (possible only with few workgroups, e.g. a
// partly resident grid).  Such a workgroup does not wait: it leaves P to the fix-up launch and
// goes on to D, so the waits cannot form a cycle.
__global__ __launch_bounds__(256, 1) void gmsq_decode_kernel(const GemmArgs a)
{
    __shared__ int red[3][4][16][64];      // partial sums handed to the wave that owns them (48 KiB)
    __shared__ float park[4][4][8][2][16]; // the deferred tile's activations (lanes c < 8; 16 KiB)
    __shared__ u32 next_t, pend_t;
    const int ntl = a.ntiles;
    const int count = a.gt.n_groups * ntl;
    u32* ticket = a.epi.status + 16;  // the ticket lives in the status block, after the word
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int q = lane >> 4, c = lane & 15;
    if (threadIdx.x == 0) next_t = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    int t = (int)next_t;
    __syncthreads();  // every wave has read next_t before thread 0 rewrites it (an empty expert's
                      // iteration has no barrier of its own)
    int pg = -1, pct = 0, pr0 = 0, pr1 = 0;  // the deferred tile
    while (t < count) {
        // draw the next ticket now; its result is needed only after this tile
        u32 nt_pending = 0;
        if (threadIdx.x == 0) nt_pending = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int g = t / ntl, ct = t % ntl;
        const int r0 = g ? a.gt.row_end[g - 1] : 0;
        const int r1 = a.gt.row_end[g];
        if (r0 < r1) {
            float act[2][16];
            u32 rmax[2];
            decode_tile_act(a, g, ct, r0, r1, red, act, rmax);
            decode_publish(a, ct, r0, r1, rmax);
            if (pg >= 0) {
                // the ticket drawn at this tile's start (returned by now) decides whether waiting
                // for the deferred tile could wait for this workgroup itself
                if (threadIdx.x == 0) pend_t = nt_pending;
                __syncthreads();
                const int pend = (int)pend_t;
                const bool self_dep = pend < count && pend / ntl == pg;
                float pact[2][16];
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int j = 0; j < 16; ++j) pact[rb][j] = c < 8 ? park[wave][q][c & 7][rb][j] : 0.0f;
                decode_finish(a, pg, pct, pr0, pr1, pact, self_dep);
            }
            if (c < 8) {
#pragma unroll
                for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                    for (int j = 0; j < 16; ++j) park[wave][q][c][rb][j] = act[rb][j];
            }
            pg = g;
            pct = ct;
            pr0 = r0;
            pr1 = r1;
        }
        if (threadIdx.x == 0) next_t = nt_pending;
        __syncthreads();
        t = (int)next_t;
        __syncthreads();  // next_t is rewritten by the next draw
    }
    if (pg >= 0) {
        float pact[2][16];
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int j = 0; j < 16; ++j) pact[rb][j] = c < 8 ? park[wave][q][c & 7][rb][j] : 0.0f;
        decode_finish(a, pg, pct, pr0, pr1, pact);
    }
}

// Fix-up launch: tiles marked in redo[g * ntiles + ct], recomputed with the final row maxima.
__global__ __launch_bounds__(256, 1) void gmsq_decode_fixup_kernel(const GemmArgs a)
{
    __shared__ int red[3][4][16][64];
    // no wait timed out in the main launch (status word 0): nothing is marked
    if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(a.epi.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0)
        return;
    const int total = a.gt.n_groups * a.ntiles;
    for (int t = blockIdx.x; t < total; t += gridDim.x) {
        if (__builtin_amdgcn_readfirstlane(__hip_atomic_load(a.epi.redo + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0)
            continue;
        const int g = t / a.ntiles, ct = t % a.ntiles;
        const int r0 = g ? a.gt.row_end[g - 1] : 0;
        const int r1 = a.gt.row_end[g];
        float act[2][16];
        u32 rmax[2];
        decode_tile_act(a, g, ct, r0, r1, red, act, rmax);
        float am[2];
        (void)decode_gather(a, r0, r1, am);  // every slot was written before this launch
        decode_tile_quant(a, ct, r0, r1, act, am);
        __syncthreads();
    }
}

}  // namespace cb
