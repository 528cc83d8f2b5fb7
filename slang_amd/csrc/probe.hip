// Roofline probes: the measured denominators the attention kernels are judged against, on the
// GPU they run on, beside the published peaks (8 TB/s HBM3E, 2.5 PFLOP/s dense f16 MFMA).
//
//   g4a_probe_read  streams a buffer once with 16-byte non-temporal buffer loads (the decode
//                   kernels' K/V stream) and folds every word into one value per workgroup, so
//                   nothing is dead: the time of a cold read of `bytes` bytes, i.e. what any
//                   kernel that must read that much from HBM costs at best.
//   g4a_probe_mfma  v_mfma_f32_32x32x16_f16 back to back from registers, 8 independent
//                   accumulator chains a wave, 2 waves a SIMD on every CU: the MFMA rate the
//                   prefill kernels' instruction could reach with no operand traffic at all.
#include "common.hpp"

namespace g4a {

typedef float float16p __attribute__((ext_vector_type(16)));
typedef unsigned u32x4_probe __attribute__((ext_vector_type(4)));
constexpr int kProbeGrid = 4096;  // most workgroups either probe launches

// workgroup w reads chunks w, w + grid, ... of 16 bytes x 256 threads (4 KiB), 8 in flight a
// thread; the per-thread XOR of every word is reduced to one word per workgroup in `sink`
__global__ __launch_bounds__(256) void probe_read_kernel(const void* p, uint32_t bytes, unsigned* sink) {
    const rsrc_t r = make_rsrc(p, bytes);
    const uint32_t stride = gridDim.x * 4096u;
    unsigned x = 0;
    for (uint32_t base = blockIdx.x * 4096u; base < bytes; base += 8 * stride) {
        u32x4_probe v[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
            v[k] = __builtin_bit_cast(u32x4_probe, __builtin_amdgcn_raw_buffer_load_b128(
                                                       r, (int)(base + k * stride + 16u * threadIdx.x), 0, kCpolNT));
#pragma unroll
        for (int k = 0; k < 8; ++k) x ^= v[k][0] ^ v[k][1] ^ v[k][2] ^ v[k][3];
    }
    __shared__ unsigned red[4];
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x ^= (unsigned)__shfl_xor((int)x, o);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

// 8 independent 32x32x16 accumulator chains a wave, `iters` rounds; the operands are
// loop-invariant registers made from the lane index, the results folded into `sink` so the
// MFMAs stay live (one float a wave)
__global__ __launch_bounds__(512) void probe_mfma_kernel(int iters, float* sink) {
    const int lane = threadIdx.x & 63;
    half8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (half_t)(0.001f * (float)((lane + i) & 7));
        b[i] = (half_t)(0.002f * (float)((lane * 3 + i) & 7));
    }
    float16p acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = float16p{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[j], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 16; ++i) s += acc[j][i];
    s = wave_sum(s);
    if (lane == 0) sink[blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)] = s;
}

}  // namespace g4a

using namespace g4a;

extern "C" size_t g4a_probe_sink_bytes(void) { return (size_t)kProbeGrid * 8 * sizeof(float); }

extern "C" int g4a_probe_read(const void* p, size_t bytes, int workgroups, void* sink, void* stream) {
    if (!p || !sink || bytes == 0 || bytes % 4096 || bytes > 0x80000000ull || ((uintptr_t)p & 15) ||
        workgroups < 0 || workgroups > kProbeGrid) {
        set_error("probe_read: p and sink non-NULL, p 16-byte aligned, bytes a multiple of 4096 up to 2 GiB, "
                  "0..%d workgroups", kProbeGrid);
        return G4A_EINVAL;
    }
    // workgroups 0: 2048, enough to keep every CU streaming; never one without a chunk to read
    const uint32_t chunks = (uint32_t)(bytes / 4096), want = workgroups ? (uint32_t)workgroups : 2048u;
    const uint32_t grid = chunks < want ? chunks : want;
    hipLaunchKernelGGL(probe_read_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, p, (uint32_t)bytes,
                       (unsigned*)sink);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? G4A_OK : hip_error(e, "probe_read launch");
}

extern "C" int g4a_probe_mfma(int workgroups, int iters, void* sink, void* stream) {
    if (!sink || workgroups <= 0 || workgroups > kProbeGrid || iters <= 0) {
        set_error("probe_mfma: sink non-NULL, 1..%d workgroups, iters > 0", kProbeGrid);
        return G4A_EINVAL;
    }
    hipLaunchKernelGGL(probe_mfma_kernel, dim3(workgroups), dim3(512), 0, (hipStream_t)stream, iters, (float*)sink);
    hipError_t e = hipGetLastError();
    return e == hipSuccess ? G4A_OK : hip_error(e, "probe_mfma launch");
}
