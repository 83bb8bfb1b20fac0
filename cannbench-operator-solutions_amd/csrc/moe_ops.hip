// moe_ops.hip - C ABI entry points of the grouped / dense int8 GEMM operators:
//   cb_grouped_matmul_swiglu_quant  (GroupedMatmulSwigluQuant)
//   cb_grouped_matmul_quant         (int8 grouped down-projection)
//   cb_quant_matmul                 (QuantMatmul)
// plus the status strings.  Each entry point validates in the reference plugin's order, then
// enqueues its kernels on the caller's stream without any allocation or host synchronisation.
#include <cstring>
#include <cstdlib>
#include <mutex>
#include <set>
#include <utility>

#include "gmsq_decode.hpp"
#include "gmsq_prefill.hpp"
#include "gemm_pf.hpp"

namespace cb {

__global__ void fill_u32_kernel(u32* p, int64_t n, u32 v)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = v;
}

static void fill_u32(u32* p, int64_t n, u32 v, hipStream_t st)
{
    int64_t blocks = (n + 255) / 256;
    blocks = blocks > 1024 ? 1024 : (blocks < 1 ? 1 : blocks);
    hipLaunchKernelGGL(fill_u32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, n, v);
}

static inline int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

// Workspace layout of GroupedMatmulSwigluQuant (all u32): the row |act| maxima (prefill: one per
// row, M words; decode: one marked slot per (row, 128-column tile), at most 32 E rows x ntiles),
// arrival counters (prefill: one per exchange round, at most M / 256 + E + 2), the status word and
// the decode kernel's tile tickets (256 bytes), then the fix-up marks (prefill: one per 256-row x
// 128-column tile; decode: one per (expert, column tile)).  No intermediate product or activation
// is ever stored: M = 131072 rows need about 0.7 MB.
struct GmsqWorkspace {
    int64_t amax_off, arrive_off, status_off, redo_off, total, n_arrive, n_redo;
};

static GmsqWorkspace gmsq_workspace(int64_t M, int64_t N, int64_t E)
{
    GmsqWorkspace w;
    const int64_t H = N / 2;
    const int64_t ntl = (H + 127) / 128;
    const int64_t dec_rows = M < 32 * E ? M : 32 * E;  // decode-shaped groups hold at most 32 rows
    const int64_t n_amax = M > dec_rows * ntl ? M : dec_rows * ntl;
    w.n_arrive = M / 256 + E + 2;
    w.n_redo = (M / 256 + E) * ntl;
    w.amax_off = 0;
    w.arrive_off = round_up(n_amax * 4, 256);
    w.status_off = w.arrive_off + round_up(w.n_arrive * 4, 256);
    w.redo_off = w.status_off + 256;
    w.total = w.redo_off + round_up(w.n_redo * 4, 256);
    return w;
}

// Compute units of the current device (cached per device): the persistent fused kernel keeps one
// workgroup per CU.
static int device_cus()
{
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    if (cus[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) v = -1;
        cus[dev] = v;
    }
    return cus[dev];
}

thread_local TestOverrides g_overrides;

// Workgroups of the persistent dequant / int32 GEMM: one per CU, unless a test forces a small grid
// (every workgroup then walks many tiles) or turns the persistent launch off.
static int persistent_grid()
{
    if (g_overrides.persistent_grid != 0) return g_overrides.persistent_grid;
    return device_cus();
}

// Polls of the GroupedMatmulSwigluQuant exchange wait before a tile gives up (each poll sleeps about
// 512 cycles plus an atomic round trip: about 2 s in total, against microseconds normally).  A tile
// that gives up is recomputed by the fix-up launch, so the limit bounds the wait, not correctness.
static constexpr int kExchangeSpins = 1 << 20;

// Raise a kernel's dynamic LDS limit once per (kernel, device): the attribute belongs to the
// kernel as loaded on the current device, so a process driving several GPUs sets it on each.
static void allow_dynamic_lds(const void* kern, int bytes)
{
    static std::mutex mu;
    static std::set<std::pair<const void*, int>> done;
    int dev = -1;
    (void)hipGetDevice(&dev);
    std::lock_guard<std::mutex> lock(mu);
    if (done.insert({kern, dev}).second)
        (void)hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

static constexpr int kSkinnyMaxRows = 32;  // groups up to this many rows take the skinny core
// The LDS core for prefill / dense groups: 256 x 256 tiles, 8 waves of 64 x 128, a 2-stage ring of
// 128-deep stages.
static constexpr int kLdsWM = 4, kLdsWN = 2, kLdsStages = 2, kLdsBK = 128;

thread_local KernelTiming g_timing;

// XCD split of the skinny kernels: the most XCDs per group (4, 2, 1) that divide the column tiles
// and still give each XCD runs of at least 1 KB per weight row (measured best: decode 2,
// down-projection 4); 0 keeps the plain block order.
static int xcd_split(int ntiles, int64_t E, int64_t tile_row_bytes)
{
    for (int P = 4; P >= 1; P >>= 1)
        if (ntiles % P == 0 && E % (8 / P) == 0 && (ntiles / P) * tile_row_bytes >= 1024) return P;
    return 0;
}

template <int EPI>
static void launch_gemm(GemmArgs& a, const int64_t* gl, int64_t E, int64_t batch, bool fast, hipStream_t st)
{
    TimedLaunch timed(st);
    static_assert(EPI == EPI_DEQUANT || EPI == EPI_I32, "GroupedMatmulSwigluQuant has its own kernels");
    const int64_t Ncols = a.N;  // output columns
    using Cfg = LdsCfg<kLdsWM, kLdsWN, kLdsStages, kLdsBK>;
    build_group_table(a.gt, gl, E, Cfg::BM);
    if (!fast) {
        a.ntiles = (int)((Ncols + 255) / 256);
        const int64_t vblocks = a.M * a.ntiles;  // the kernels loop over virtual blocks past the grid
        const dim3 grid((unsigned)(vblocks < (1 << 20) ? vblocks : (1 << 20)), (unsigned)batch);
        if constexpr (EPI == EPI_I32)
            hipLaunchKernelGGL(generic_i32_kernel, grid, dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL(generic_dequant_kernel, grid, dim3(256), 0, st, a);
        return;
    }
    if (a.gt.max_rows <= kSkinnyMaxRows) {
        a.ntiles = (int)((Ncols + 255) / 256);
        const dim3 grid((unsigned)a.ntiles, (unsigned)E, (unsigned)batch);
        // XCD split: the most XCDs per group (4, 2, 1) that divide the column tiles and still give
        // each XCD runs of at least 1 KB per weight row (measured best: decode 2, down-projection 4)
        a.xcd_split = 0;
        if (batch == 1) {
            a.xcd_split = xcd_split(a.ntiles, E, 256);
        }
        hipLaunchKernelGGL((skinny_kernel<EPI>), grid, dim3(256), 0, st, a);
        return;
    }
    a.ntiles = (int)((Ncols + 255) / 256);
    const int64_t blocks = (int64_t)a.gt.total_mtiles * a.ntiles;
    const int pg = persistent_grid();
    if constexpr (EPI == EPI_DEQUANT) {
        // the four-wave ring core with a continuous stage stream (K of at least 4 stages) and
        // 16-byte stores of 8 columns (N a multiple of 8, the output 16-byte aligned)
        if (batch == 1 && pg > 0 && a.K >= 4 * PfCfg::BK && Ncols % 8 == 0 && aligned(a.epi.out, 16) &&
            256 * Ncols * 2 < 0x7fffffffLL) {
            const EpiArgs& e = a.epi;
            const bool simple = !e.has_offset && e.bias_kind == BIAS_NONE && e.out_bf16;
            const void* kern = simple ? (const void*)gpf_dequant_kernel<true> : (const void*)gpf_dequant_kernel<false>;
            allow_dynamic_lds(kern, kGpfLds);
            // the block map's valid slots are spread over each round of 256: launch the whole grid
            const bool bm = gpf_block_map(a.gt.total_mtiles, a.ntiles);
            const dim3 grid((unsigned)(bm || blocks > pg ? pg : blocks));
            if (simple) hipLaunchKernelGGL(gpf_dequant_kernel<true>, grid, dim3(256), kGpfLds, st, a);
            else hipLaunchKernelGGL(gpf_dequant_kernel<false>, grid, dim3(256), kGpfLds, st, a);
            return;
        }
    }
    // persistent launch once there are more tiles than workgroups (one continuous DMA stream per
    // workgroup: a tile's last STAGES iterations issue the next tile's first STAGES stages, so K
    // must span at least STAGES stages); its register-direct epilogue addresses a tile's rows with
    // 32-bit offsets
    if (batch == 1 && pg > 0 && blocks > pg && a.K >= (int64_t)Cfg::STAGES_ * Cfg::BK &&
        Cfg::BM * Ncols * 4 < 0x7fffffffLL) {
        auto kern = lds_gemm_persistent_kernel<EPI, kLdsWM, kLdsWN, kLdsStages, kLdsBK>;
        constexpr int lds = Cfg::CONT_LDS_BYTES;  // the ring and two row-scale slots
        allow_dynamic_lds((const void*)kern, lds);
        hipLaunchKernelGGL(kern, dim3((unsigned)pg), dim3(Cfg::NT), lds, st, a);
        return;
    }
    auto kern = lds_gemm_kernel<EPI, kLdsWM, kLdsWN, kLdsStages, kLdsBK>;
    allow_dynamic_lds((const void*)kern, Cfg::LDS_BYTES);
    hipLaunchKernelGGL(kern, dim3((unsigned)blocks, (unsigned)batch), dim3(Cfg::NT), Cfg::LDS_BYTES, st, a);
}

}  // namespace cb

using namespace cb;

extern "C" const char* cb_status_string(int s)
{
    switch (s) {
        case CB_OK: return "ok";
        case CB_ERR_NULL_POINTER: return "a required tensor pointer is NULL";
        case CB_ERR_DTYPE: return "unsupported dtype";
        case CB_ERR_SHAPE: return "invalid or unsupported shape";
        case CB_ERR_K_MISMATCH: return "K mismatch between x and weight";
        case CB_ERR_N_ODD: return "N must be even";
        case CB_ERR_GROUP_LEN: return "group_list length must equal the expert count";
        case CB_ERR_GROUP_COUNT: return "unsupported expert count";
        case CB_ERR_GROUP_ORDER: return "group_list must be a cumsum <= M";
        case CB_ERR_GROUP_TOTAL: return "group_list[-1] must equal M";
        case CB_ERR_SCALE_LEN: return "scale / offset / pertoken / bias length mismatch";
        case CB_ERR_ROW_TOO_LONG: return "row length must not exceed 16384";
        case CB_ERR_WORKSPACE: return "workspace missing or too small";
        case CB_ERR_EMPTY: return "non-empty shapes required";
        case CB_ERR_LAUNCH: return "HIP kernel launch failed";
        case CB_ERR_NO_DEVICE: return "no usable gfx950 device";
        case CB_ERR_SCRATCH_LIMIT: return "problem exceeds the fixed scratch of the no-allocation entry point";
        default: return "unknown status";
    }
}

extern "C" const char* cb_version(void) { return "cannbench_amd 0.1 gfx950"; }

extern "C" void cb_set_kernel_timing(void* start_event, void* stop_event)
{
    g_timing.start = (hipEvent_t)start_event;
    g_timing.stop = (hipEvent_t)stop_event;
}

extern "C" int64_t cb_grouped_matmul_swiglu_quant_workspace_size(int64_t M, int64_t K, int64_t N, int64_t E)
{
    (void)K;
    (void)E;
    if (M <= 0 || N <= 0) return 0;
    return gmsq_workspace(M, N, E).total;
}

// GroupedMatmulSwigluQuant, optionally with the activation rows gathered through row_index (x then
// holds x_rows rows, x_scale x_rows scales).
static int gmsq_impl(const int8_t* x, int64_t x_rows, const int32_t* row_index, const int8_t* weight,
                     const float* weight_scale, const float* x_scale, const int64_t* group_list,
                     int64_t group_len, int64_t M, int64_t K, int64_t N, int64_t E, int8_t* y,
                     float* y_scale, void* workspace, int64_t workspace_bytes, void* stream)
{
    if (M < 0 || K < 0 || N < 0 || E < 0 || x_rows < 0) return CB_ERR_SHAPE;
    if (N % 2 != 0) return CB_ERR_N_ODD;  // GmsqMeta checks this before anything else
    if (M == 0 || N == 0 || E == 0) return CB_OK;  // gmsq_plugin.cpp:93-95
    if (!x || !weight || !weight_scale || !x_scale || !y || !y_scale) return CB_ERR_NULL_POINTER;
    if (M > 0x7fffffffLL) return CB_ERR_SHAPE;
    // gathered rows are addressed with 32-bit offsets into x
    if (row_index && (x_rows == 0 || x_rows * K >= 0x7fffffffLL)) return CB_ERR_SHAPE;
    const int vs = validate_group_list(group_list, group_len, E, M);
    if (vs != CB_OK) return vs;
    const GmsqWorkspace ws = gmsq_workspace(M, N, E);
    if (!workspace || workspace_bytes < ws.total) return CB_ERR_WORKSPACE;

    hipStream_t st = (hipStream_t)stream;
    const int64_t H = N / 2;
    uint8_t* wsb = (uint8_t*)workspace;
    u32* amax = (u32*)(wsb + ws.amax_off);

    GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = x;
    a.w = weight;
    a.M = M;
    a.K = K;
    a.N = N;
    a.w_gstride = K * N;
    a.row_index = row_index;
    a.x_rows = row_index ? x_rows : M;
    a.epi.w_scale = weight_scale;
    a.epi.x_scale = x_scale;
    a.epi.amax = amax;
    a.epi.H = H;
    a.epi.arrive = (u32*)(wsb + ws.arrive_off);
    a.epi.status = (u32*)(wsb + ws.status_off);
    a.epi.redo = (u32*)(wsb + ws.redo_off);
    a.epi.yq = y;
    a.epi.yq_scale = y_scale;
    a.epi.spin_limit = g_overrides.exchange_spin_limit != 0 ? g_overrides.exchange_spin_limit : kExchangeSpins;
    build_group_table(a.gt, group_list, E, 256);
    // row maxima, arrival counters, the status word and the fix-up marks are contiguous: one fill
    // clears what this call's launches use
    auto clear_ws = [&](int64_t n_redo) { fill_u32(amax, (ws.redo_off - ws.amax_off) / 4 + n_redo, 0u, st); };

    const bool fast = K > 0 && K % 16 == 0 && H % 16 == 0 && offsets32_ok(K, N) && aligned(x, 16) &&
                      aligned(weight, 16) && aligned(weight_scale, 4);
    const int ntl = (int)((H + 127) / 128);  // 128-act-column tiles
    // a test that turns the persistent launches off also takes the two-pass path here: the path
    // taken when the fused kernels' grids cannot all be resident
    const bool fused = g_overrides.persistent_grid >= 0;
    if (fused && fast && a.gt.max_rows > kSkinnyMaxRows) {
        // (y at any alignment: the stores narrow to bytes when y is not 4-byte aligned)
        // prefill-shaped groups: the persistent GEMM with the requant fused
        const int cus = device_cus();
        const int grid = (ntl == 16 && cus >= 256) ? 256 : (cus / ntl) * ntl;
        const bool gather = row_index != nullptr;
        const bool defer = (K + PfCfg::BK - 1) / PfCfg::BK >= kPfDeferMinStages;
        const void* main_k = gather ? (defer ? (const void*)gmsq_prefill_kernel<true, true>
                                             : (const void*)gmsq_prefill_kernel<true, false>)
                                    : (defer ? (const void*)gmsq_prefill_kernel<false, true>
                                             : (const void*)gmsq_prefill_kernel<false, false>);
        const void* fix_k =
            gather ? (const void*)gmsq_prefill_fixup_kernel<true> : (const void*)gmsq_prefill_fixup_kernel<false>;
        int resident = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, main_k, 256, kPfLds) != hipSuccess) resident = 0;
        // every workgroup of an exchange group must be resident at once: one per CU at most
        if (grid >= ntl && resident >= 1 && a.gt.total_mtiles + 2 <= ws.n_arrive) {
            a.ntiles = ntl;
            clear_ws((int64_t)a.gt.total_mtiles * ntl);
            allow_dynamic_lds(main_k, kPfLds);
            allow_dynamic_lds(fix_k, kPfLds);
            const int tiles = a.gt.total_mtiles * ntl;
            const dim3 fix_grid((unsigned)(tiles < 256 ? tiles : 256));
            {
                TimedLaunch timed(st);
                void* args[] = {(void*)&a};
                (void)hipLaunchKernel(main_k, dim3((unsigned)grid), dim3(256), args, kPfLds, st);  // checked below
            }
            if (gather) hipLaunchKernelGGL(gmsq_prefill_fixup_kernel<true>, fix_grid, dim3(256), kPfLds, st, a);
            else hipLaunchKernelGGL(gmsq_prefill_fixup_kernel<false>, fix_grid, dim3(256), kPfLds, st, a);
            return check_launch();
        }
    }
    if (fused && fast && a.gt.max_rows <= kSkinnyMaxRows) {
        // (y at any alignment: 16-byte, dword or byte stores by the alignment of y)
        // decode-shaped groups: weight streaming with the requant fused (per-expert exchange), on a
        // persistent grid of one workgroup per CU (each wave keeps two weight chunks in flight in
        // its registers) drawing tiles from one ticket in expert order
        const int cus = device_cus();
        int resident = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, (const void*)gmsq_decode_kernel, 256, 0) !=
            hipSuccess)
            resident = 0;
        const int64_t tiles = E * ntl;
        int grid = (resident < 1 ? resident : 1) * cus;
        if (g_overrides.persistent_grid > 0 && resident >= 1) grid = g_overrides.persistent_grid;  // test hook
        if (grid > tiles) grid = (int)tiles;
        if (grid >= 1) {
            a.ntiles = ntl;
            clear_ws(tiles);
            {
                TimedLaunch timed(st);
                hipLaunchKernelGGL(gmsq_decode_kernel, dim3((unsigned)grid), dim3(256), 0, st, a);
            }
            hipLaunchKernelGGL(gmsq_decode_fixup_kernel, dim3((unsigned)(tiles < 512 ? tiles : 512)), dim3(256), 0, st, a);
            return check_launch();
        }
    }
    // any other shape or alignment: two passes over the products (row maxima, then the requant)
    clear_ws(0);
    a.ntiles = (int)((H + 255) / 256);
    const int64_t vblocks = M * a.ntiles;  // the kernels loop over virtual blocks past the grid
    const dim3 grid((unsigned)(vblocks < (1 << 20) ? vblocks : (1 << 20)));
    {
        TimedLaunch timed(st);
        hipLaunchKernelGGL(generic_swiglu_kernel<false>, grid, dim3(256), 0, st, a);
    }
    hipLaunchKernelGGL(generic_swiglu_kernel<true>, grid, dim3(256), 0, st, a);
    return check_launch();
}

extern "C" int cb_grouped_matmul_swiglu_quant(const int8_t* x, const int8_t* weight, const float* weight_scale,
                                              const float* x_scale, const int64_t* group_list,
                                              int64_t group_len, int64_t M, int64_t K, int64_t N, int64_t E,
                                              int8_t* y, float* y_scale, void* workspace,
                                              int64_t workspace_bytes, void* stream)
{
    return gmsq_impl(x, M, nullptr, weight, weight_scale, x_scale, group_list, group_len, M, K, N, E, y, y_scale,
                     workspace, workspace_bytes, stream);
}

extern "C" int cb_grouped_matmul_swiglu_quant_gather(const int8_t* x, int64_t x_rows, const int32_t* row_index,
                                                     const int8_t* weight, const float* weight_scale,
                                                     const float* x_scale, const int64_t* group_list,
                                                     int64_t group_len, int64_t M, int64_t K, int64_t N, int64_t E,
                                                     int8_t* y, float* y_scale, void* workspace,
                                                     int64_t workspace_bytes, void* stream)
{
    if (!row_index && M > 0 && N > 0 && E > 0) return CB_ERR_NULL_POINTER;
    return gmsq_impl(x, x_rows, row_index, weight, weight_scale, x_scale, group_list, group_len, M, K, N, E, y,
                     y_scale, workspace, workspace_bytes, stream);
}

// The fixed workspace of cb_grouped_matmul_swiglu_quant_noalloc: one array per GPU (each device
// holds its own copy of a __device__ variable).  Host code uses the address looked up on each
// device, never the array's name.
static constexpr int64_t kNoAllocScratchBytes = 4 << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// Device address of `scratch` on the current device, looked up once per device.
static void* noalloc_scratch(int* status)
{
    static std::mutex mu;
    static void* ptrs[64] = {nullptr};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        *status = CB_ERR_NO_DEVICE;
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            *status = CB_ERR_NO_DEVICE;
            return nullptr;
        }
        ptrs[dev] = p;
    }
    *status = CB_OK;
    return ptrs[dev];
}

extern "C" int cb_grouped_matmul_swiglu_quant_noalloc(const int8_t* x, const int8_t* weight,
                                                      const float* weight_scale, const float* x_scale,
                                                      const int64_t* group_list, int64_t group_len, int64_t M,
                                                      int64_t K, int64_t N, int64_t E, int8_t* y, float* y_scale,
                                                      void* stream)
{
    // the checks that come before any workspace use, in the order of the workspace entry point
    if (M < 0 || K < 0 || N < 0 || E < 0) return CB_ERR_SHAPE;
    if (N % 2 != 0) return CB_ERR_N_ODD;
    if (M == 0 || N == 0 || E == 0) return CB_OK;
    if (gmsq_workspace(M, N, E).total > kNoAllocScratchBytes) return CB_ERR_SCRATCH_LIMIT;
    int rc = CB_OK;
    void* ws = noalloc_scratch(&rc);
    if (rc != CB_OK) return rc;
    return gmsq_impl(x, M, nullptr, weight, weight_scale, x_scale, group_list, group_len, M, K, N, E, y, y_scale, ws,
                     kNoAllocScratchBytes, stream);
}

extern "C" int cb_grouped_matmul_swiglu_quant_status(const void* workspace, int64_t M, int64_t N, int64_t E,
                                                     uint32_t* status, void* stream)
{
    if (!workspace || !status) return CB_ERR_NULL_POINTER;
    if (M <= 0 || N <= 0 || E <= 0) {
        *status = 0;  // no launch happened
        return CB_OK;
    }
    const GmsqWorkspace ws = gmsq_workspace(M, N, E);
    hipStream_t st = (hipStream_t)stream;
    if (hipMemcpyAsync(status, (const uint8_t*)workspace + ws.status_off, 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return CB_ERR_LAUNCH;
    return CB_OK;
}

extern "C" int cb_grouped_matmul_quant(const int8_t* x, const int8_t* weight, const float* weight_scale,
                                       const float* x_scale, const int64_t* group_list, int64_t group_len,
                                       int64_t M, int64_t K, int64_t N, int64_t E, void* out, void* stream)
{
    if (M < 0 || K < 0 || N < 0 || E < 0) return CB_ERR_SHAPE;
    if (E < 1) return CB_ERR_GROUP_COUNT;  // grouped_matmul_plugin.cpp:133
    if (M == 0 || N == 0) {
        const int vs = validate_group_list(group_list, group_len, E, M);
        return vs;
    }
    if (!x || !weight || !weight_scale || !x_scale || !out) return CB_ERR_NULL_POINTER;
    if (M > 0x7fffffffLL) return CB_ERR_SHAPE;
    const int vs = validate_group_list(group_list, group_len, E, M);
    if (vs != CB_OK) return vs;

    GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = x;
    a.w = weight;
    a.M = M;
    a.K = K;
    a.N = N;
    a.w_gstride = K * N;
    a.epi.scale = weight_scale;
    a.epi.scale_gstride = N;
    a.epi.scale_perchan = 1;
    a.epi.pertoken = x_scale;
    a.epi.has_pt = 1;
    a.epi.out = out;
    a.epi.out_bf16 = 1;
    const bool fast = K > 0 && K % 16 == 0 && N % 16 == 0 && offsets32_ok(K, N) && aligned(x, 16) &&
                      aligned(weight, 16) && aligned(out, 16);
    launch_gemm<EPI_DEQUANT>(a, group_list, E, 1, fast, (hipStream_t)stream);
    return check_launch();
}

extern "C" int cb_quant_matmul(const int8_t* x1, const int8_t* x2, const void* scale, int scale_dtype,
                               int64_t scale_numel, const float* offset, int64_t offset_numel,
                               const float* pertoken, int64_t pertoken_numel, const void* bias, int bias_dtype,
                               int64_t bias_numel, int bias_batched, int64_t batch, int64_t M, int64_t K,
                               int64_t N, int out_dtype, void* out, void* stream)
{
    // quant_matmul_plugin.cpp:86-175, in order.
    if (!x1 || !x2 || !scale) return CB_ERR_NULL_POINTER;
    if (scale_dtype != CB_DT_FLOAT32 && scale_dtype != CB_DT_BFLOAT16) return CB_ERR_DTYPE;
    if (out_dtype != CB_DT_FLOAT16 && out_dtype != CB_DT_BFLOAT16) return CB_ERR_DTYPE;
    if (K <= 0 || M <= 0 || N <= 0) return CB_ERR_EMPTY;
    if (batch < 1 || M > 0x7fffffffLL) return CB_ERR_SHAPE;
    if (scale_numel != 1 && scale_numel != N) return CB_ERR_SCALE_LEN;
    if (offset_numel != 0) {
        if (!offset) return CB_ERR_NULL_POINTER;
        if (offset_numel != 1 && offset_numel != N) return CB_ERR_SCALE_LEN;
    }
    if (pertoken_numel != 0) {
        if (!pertoken) return CB_ERR_NULL_POINTER;
        if (pertoken_numel != M) return CB_ERR_SCALE_LEN;
    }
    int bias_kind = BIAS_NONE;
    if (bias_numel != 0) {
        if (!bias) return CB_ERR_NULL_POINTER;
        switch (bias_dtype) {
            case CB_DT_INT32: bias_kind = BIAS_I32; break;
            case CB_DT_FLOAT16: bias_kind = BIAS_F16; break;
            case CB_DT_BFLOAT16: bias_kind = BIAS_BF16; break;
            case CB_DT_FLOAT32: bias_kind = BIAS_F32; break;
            default: return CB_ERR_DTYPE;
        }
        if (bias_batched) {
            if (!(batch > 1 && bias_numel == batch * N)) return CB_ERR_SCALE_LEN;
        } else if (bias_numel != 1 && bias_numel != N) {
            return CB_ERR_SCALE_LEN;
        }
    }
    if (!out) return CB_ERR_NULL_POINTER;

    GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = x1;
    a.w = x2;
    a.M = M;
    a.K = K;
    a.N = N;
    a.x_bstride = M * K;
    a.w_bstride = K * N;
    a.w_gstride = 0;
    EpiArgs& e = a.epi;
    e.scale = scale;
    e.scale_bf16 = scale_dtype == CB_DT_BFLOAT16;
    e.scale_perchan = scale_numel > 1;
    e.offset = offset;
    e.has_offset = offset_numel != 0;
    e.offset_perchan = offset_numel > 1;
    e.pertoken = pertoken;
    e.has_pt = pertoken_numel != 0;
    e.bias = bias;
    e.bias_kind = bias_kind;
    e.bias_perchan = bias_batched ? (N > 1) : (bias_numel > 1);
    e.bias_bstride = bias_batched ? N : 0;
    e.out = out;
    e.out_bf16 = out_dtype == CB_DT_BFLOAT16;
    e.out_bstride = M * N;
    const int64_t gl[1] = {M};
    const bool fast = K % 16 == 0 && N % 16 == 0 && offsets32_ok(K, N) && aligned(x1, 16) && aligned(x2, 16) &&
                      aligned(out, 16);
    launch_gemm<EPI_DEQUANT>(a, gl, 1, batch, fast, (hipStream_t)stream);
    return check_launch();
}

extern "C" int cb_grouped_matmul_int32(const int8_t* x, const int8_t* weight, const int64_t* group_list,
                                       int64_t group_len, int64_t M, int64_t K, int64_t N, int64_t E,
                                       int32_t* c, void* stream)
{
    if (M < 0 || K < 0 || N < 0 || E < 0) return CB_ERR_SHAPE;
    if (E < 1) return CB_ERR_GROUP_COUNT;
    const int vs = validate_group_list(group_list, group_len, E, M);
    if (vs != CB_OK) return vs;
    if (M == 0 || N == 0) return CB_OK;
    if (!x || !weight || !c) return CB_ERR_NULL_POINTER;
    if (M > 0x7fffffffLL) return CB_ERR_SHAPE;
    GemmArgs a;
    std::memset(&a, 0, sizeof(a));
    a.x = x;
    a.w = weight;
    a.M = M;
    a.K = K;
    a.N = N;
    a.w_gstride = K * N;
    a.epi.out = c;
    const bool fast = K > 0 && K % 16 == 0 && N % 16 == 0 && offsets32_ok(K, N) && aligned(x, 16) &&
                      aligned(weight, 16) && aligned(c, 16);
    launch_gemm<EPI_I32>(a, group_list, E, 1, fast, (hipStream_t)stream);
    return check_launch();
}

extern "C" void cb_set_test_overrides(int persistent_grid, int exchange_spin_limit, int gmm_tile)
{
    g_overrides.persistent_grid = persistent_grid;
    g_overrides.exchange_spin_limit = exchange_spin_limit;
    g_overrides.gmm_tile = gmm_tile;
}
