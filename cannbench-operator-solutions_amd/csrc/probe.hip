// probe.hip - measurement kernel with no reference counterpart: the int8 matrix-core rate this
// device sustains, to set the GEMM figures beside.  Every CU runs waves that issue independent
// chains of v_mfma_i32_32x32x32_i8 on register operands, with no memory traffic in the loop, so
// the rate is the MFMA issue rate at the clock the part holds under that load.
#include <cstdint>

#include "common.hpp"
#include "host_util.hpp"

namespace cb {

typedef int v16i_p __attribute__((ext_vector_type(16)));

constexpr int kProbeChains = 8;  // independent accumulators per wave

__global__ __launch_bounds__(256) void mfma_probe_kernel(int64_t iters, int32_t* __restrict__ sink)
{
    const int lane = threadIdx.x & 63;
    const v4i a = {lane * 3 + 1, lane ^ 0x5a5a, 0x01020304 + lane, -lane};
    const v4i b = {0x7f7f0101 ^ lane, lane * 7, 0x10203040, lane + 11};
    v16i_p acc[kProbeChains];
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = c + r;
    for (int64_t it = 0; it < iters; ++it) {
#pragma unroll
        for (int c = 0; c < kProbeChains; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
    }
    int s = 0;
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s ^= acc[c][r];
    if (lane == 0) sink[blockIdx.x * 4 + (threadIdx.x >> 6)] = s;  // keeps the chains live
}

}  // namespace cb

using namespace cb;

extern "C" int cb_probe_mfma_i8(int64_t iters, int32_t* sink, int64_t sink_len, int64_t* ops, void* stream)
{
    if (!sink || !ops) return CB_ERR_NULL_POINTER;
    if (iters <= 0) return CB_ERR_SHAPE;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        return CB_ERR_NO_DEVICE;
    const int64_t grid = 2 * (int64_t)cus;  // 2 workgroups of 4 waves per CU: 2 waves per SIMD
    if (sink_len < grid * 4) return CB_ERR_SHAPE;
    hipStream_t st = (hipStream_t)stream;
    TimedLaunch timed(st);
    hipLaunchKernelGGL(mfma_probe_kernel, dim3((unsigned)grid), dim3(256), 0, st, iters, sink);
    *ops = grid * 4 * iters * kProbeChains * (int64_t)(2 * 32 * 32 * 32);
    return check_launch();
}
