// The rest of a layers-outer batched prefill around the attention block, for gfx950: the
// element- and row-wise tails between the f16 GEMMs of PrefillGPU._layer
// (gemma4_150/prefill_gpu.py:316-395): the residual add + RMSNorm after the o, down and
// per-layer-embedding projections fused with the norm or quantisation that makes the next
// GEMM's f16 operand (rmsadd_b + rmssrqh_b / srqh_b / rmssrq_69,
// kernels_dsl.py:622-710, 158-206, 233-242), the GeGLU tail of the gate/up GEMMs (geglu_b,
// :259-290) and the per-layer-embedding gate tail (plegate_b, :1767-1786, with the srqh_b
// that follows it at prefill_gpu.py:383-384).
//
// MI355X design: every kernel is one pass over HBM-resident [S][n] activations (row tails:
// one workgroup per token row, the row in registers; elementwise tails: 8 values per thread,
// 16-byte loads and stores). The f16 outputs are the GEMM A operands of the next step, so no
// separate conversion pass runs between them.
#include <math.h>

#include "common.hpp"

namespace g4a {

__device__ __forceinline__ float row_sum(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();  // red may still be read by a previous sum
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

struct TailArgs {
    const half_t* x16;  // [rows][n] GEMM output, or NULL: no residual add
    const float* w1;
    float* hidden;      // [rows][n] in/out
    const float* w2;
    half_t* y16;        // [rows][n]
    int n, mode;
    float x_q, mult, eps, q2;
};

// Row r: d = srq(f32(x16), x_q); hidden = (hidden + d / sqrt(mean(d^2) + eps) * w1) * mult
// (rmsadd_b), then by mode the next GEMM operand y16 = f16(srq(hidden, q2)) (G4A_TAIL_SRQ,
// srqh_b), f16(srq(z, q2)) with z = hidden / sqrt(mean(hidden^2) + eps) * w2 (G4A_TAIL_NORM,
// rmssrq_69 then srqh_b) or f16(srq(f32(f16(z)), q2)) (G4A_TAIL_NORM16, rmssrqh_b's double
// rounding). Thread t holds elements t + 256k.
template <int PER>
__global__ __launch_bounds__(256) void rows_tail_kernel(TailArgs a) {
    __shared__ float red[4];
    const size_t base = (size_t)blockIdx.x * a.n;
    float h[PER], d[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = threadIdx.x + 256 * k;
        const bool ok = i < a.n;
        h[k] = ok ? a.hidden[base + i] : 0.0f;
        d[k] = ok && a.x16 ? srq((float)a.x16[base + i], a.x_q) : 0.0f;
    }
    if (a.x16) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; ++k) ss = __builtin_fmaf(d[k], d[k], ss);
        const float r = sqrtf(row_sum(ss, red) / (float)a.n + a.eps);
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = threadIdx.x + 256 * k;
            if (i < a.n) {
                h[k] = (h[k] + d[k] / r * a.w1[i]) * a.mult;
                a.hidden[base + i] = h[k];
            }
        }
    }
    if (a.mode == G4A_TAIL_NONE) return;
    float r2 = 1.0f;
    if (a.mode != G4A_TAIL_SRQ) {
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; ++k) ss = __builtin_fmaf(h[k], h[k], ss);
        r2 = sqrtf(row_sum(ss, red) / (float)a.n + a.eps);
    }
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = threadIdx.x + 256 * k;
        if (i >= a.n) continue;
        float z = a.mode == G4A_TAIL_SRQ ? h[k] : pin(h[k] / r2 * a.w2[i]);
        if (a.mode == G4A_TAIL_NORM16) z = (float)(half_t)z;
        a.y16[base + i] = (half_t)srq(z, a.q2);
    }
}

// The same row tail with one wave per row and 8 consecutive elements per lane and load
// (rows of n % 8 == 0 values): no barrier, 16-byte loads and stores. Lane l holds chunks
// l, l + 64, .. (J of them at most) of its row; the sums of squares run over a lane's
// elements in order, then across the wave, so they are f32 sums in another order than
// rows_tail_kernel's (the per-element arithmetic is the same).
template <int J>
__global__ __launch_bounds__(256) void rows_tail_wave_kernel(TailArgs a, int n_rows) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= n_rows) return;  // the whole wave
    const int C = a.n / 8;
    const size_t base = (size_t)row * a.n;
    float8v h[J], d[J], w1[J], w2[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {  // every operand of the row in flight at once
        const int c = lane + 64 * j;
        h[j] = d[j] = w1[j] = w2[j] = float8v{};
        if (c < C) {
            h[j] = load8(a.hidden + base + 8 * c);
            if (a.x16) {
                d[j] = load8(a.x16 + base + 8 * c);
                w1[j] = load8(a.w1 + 8 * c);
            }
            if (a.mode == G4A_TAIL_NORM || a.mode == G4A_TAIL_NORM16) w2[j] = load8(a.w2 + 8 * c);
        }
    }
    if (a.x16) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                d[j][i] = srq(d[j][i], a.x_q);
                ss = __builtin_fmaf(d[j][i], d[j][i], ss);
            }
        const float r = sqrtf(wave_sum(ss) / (float)a.n + a.eps);
#pragma unroll
        for (int j = 0; j < J; ++j) {
            const int c = lane + 64 * j;
            if (c < C) {
#pragma unroll
                for (int i = 0; i < 8; ++i) h[j][i] = (h[j][i] + d[j][i] / r * w1[j][i]) * a.mult;
                float* hp = a.hidden + base + 8 * c;
                *reinterpret_cast<float4v*>(hp) = float4v{h[j][0], h[j][1], h[j][2], h[j][3]};
                *reinterpret_cast<float4v*>(hp + 4) = float4v{h[j][4], h[j][5], h[j][6], h[j][7]};
            }
        }
    }
    if (a.mode == G4A_TAIL_NONE) return;
    float r2 = 1.0f;
    if (a.mode != G4A_TAIL_SRQ) {
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < J; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(h[j][i], h[j][i], ss);
        r2 = sqrtf(wave_sum(ss) / (float)a.n + a.eps);
    }
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int c = lane + 64 * j;
        if (c >= C) continue;
        half8 y;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float z = a.mode == G4A_TAIL_SRQ ? h[j][i] : pin(h[j][i] / r2 * w2[j][i]);
            if (a.mode == G4A_TAIL_NORM16) z = (float)(half_t)z;
            y[i] = (half_t)srq(z, a.q2);
        }
        *reinterpret_cast<half8*>(a.y16 + base + 8 * c) = y;
    }
}

// geglu_b: g = srq(f32(gate), gate_q), u = srq(f32(up), up_q), y = gelu(g) * u (gelu from the
// layer's table when given, gelu_srq); out = f16(clamp(round(y / out_q), -128, 127)) -- the code
// on out_q's grid, which the down GEMM scales back by alpha = out_q -- or f16(y) when out_q is 0.
__global__ __launch_bounds__(256) void geglu16_kernel(int n8, const half8* gate, const half8* up, float gq, float uq,
                                                      float oq, half8* out, const float* lut) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const half8 g = gate[i], u = up[i];
    half8 o;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = geglu_code((float)g[j], (float)u[j], gq, uq, oq, lut);
    out[i] = o;
}

// plegate_b + srqh_b: out[s][o] = f16(srq(gelu(srq(f32(lin[s][o]), lin_q)) * ple[s*stride + o], out_q)),
// d values per row (a multiple of 8); gelu from the layer's table when given (gelu_srq).
__global__ __launch_bounds__(256) void plegate16_kernel(int n8, int d, const half8* lin, float lq, const float* ple,
                                                        int stride, float oq, half8* out, const float* lut) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const int s = (8 * i) / d, o = (8 * i) % d;
    const half8 x = lin[i];
    const float* pr = ple + (size_t)s * stride + o;
    const float4v p0 = *reinterpret_cast<const float4v*>(pr), p1 = *reinterpret_cast<const float4v*>(pr + 4);
    const float pv[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
    half8 y;
#pragma unroll
    for (int j = 0; j < 8; ++j) y[j] = (half_t)srq(pin(gelu_srq(srq((float)x[j], lq), lq, lut) * pv[j]), oq);
    out[i] = y;
}

}  // namespace g4a

using namespace g4a;

extern "C" int g4a_rows_tail(int n_rows, int n, const void* x16, float x_q, const float* w1, float mult, float eps,
                             float* hidden, int mode, const float* w2, float q2, void* y16, void* stream) {
    if (n_rows <= 0 || n <= 0 || n > 4096) {
        set_error("n_rows (%d) must be positive and n (%d) in [1, 4096]", n_rows, n);
        return G4A_EINVAL;
    }
    if (mode < G4A_TAIL_NONE || mode > G4A_TAIL_NORM16) {
        set_error("mode %d unknown", mode);
        return G4A_EINVAL;
    }
    if (!hidden || (x16 && !w1) || (mode != G4A_TAIL_NONE && !y16) ||
        ((mode == G4A_TAIL_NORM || mode == G4A_TAIL_NORM16) && !w2) || (!x16 && mode == G4A_TAIL_NONE)) {
        set_error("hidden non-NULL; w1 with x16; y16 unless mode is NONE; w2 for the norm modes; x16 or a mode");
        return G4A_EINVAL;
    }
    if (!(x_q >= 0.0f) || !(q2 >= 0.0f) || !(eps >= 0.0f)) {
        set_error("x_q, q2 and eps must be >= 0");
        return G4A_EINVAL;
    }
    TailArgs a;
    a.x16 = reinterpret_cast<const half_t*>(x16);
    a.w1 = w1;
    a.hidden = hidden;
    a.w2 = w2;
    a.y16 = reinterpret_cast<half_t*>(y16);
    a.n = n;
    a.mode = mode;
    a.x_q = x_q;
    a.mult = mult;
    a.eps = eps;
    a.q2 = q2;
    const bool vec = n % 8 == 0 && !(((uintptr_t)hidden | (uintptr_t)x16 | (uintptr_t)w1 | (uintptr_t)w2 |
                                       (uintptr_t)y16) & 15);
    if (vec) {  // one wave per row: the 1024-token decoder prefill (106 row tails) 8.52 -> 8.36 ms
        const int J = (n / 8 + 63) / 64;
        auto fn = J <= 1 ? rows_tail_wave_kernel<1> : J <= 2 ? rows_tail_wave_kernel<2>
                : J <= 3 ? rows_tail_wave_kernel<3> : J <= 4 ? rows_tail_wave_kernel<4> : rows_tail_wave_kernel<8>;
        hipLaunchKernelGGL(fn, dim3((n_rows + 3) / 4), dim3(256), 0, (hipStream_t)stream, a, n_rows);
    } else {
        const int per = (n + 255) / 256;
        auto fn = per <= 2 ? rows_tail_kernel<2> : per <= 4 ? rows_tail_kernel<4> : per <= 8 ? rows_tail_kernel<8>
                                                                                           : rows_tail_kernel<16>;
        hipLaunchKernelGGL(fn, dim3(n_rows), dim3(256), 0, (hipStream_t)stream, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "rows_tail launch");
    return G4A_OK;
}

extern "C" int g4a_geglu16(int n, const void* gate16, const void* up16, float gate_q, float up_q, float out_q,
                           void* out16, const float* gelu_lut, void* stream) {
    if (n <= 0 || n % 8 || !gate16 || !up16 || !out16 ||
        (((uintptr_t)gate16 | (uintptr_t)up16 | (uintptr_t)out16) & 15)) {
        set_error("n (%d) a positive multiple of 8; gate, up, out non-NULL and 16-byte aligned", n);
        return G4A_EINVAL;
    }
    if (!(gate_q >= 0.0f) || !(up_q >= 0.0f) || !(out_q >= 0.0f)) {
        set_error("gate_q, up_q and out_q must be >= 0");
        return G4A_EINVAL;
    }
    const int n8 = n / 8;
    hipLaunchKernelGGL(geglu16_kernel, dim3((n8 + 255) / 256), dim3(256), 0, (hipStream_t)stream, n8,
                       reinterpret_cast<const half8*>(gate16), reinterpret_cast<const half8*>(up16), gate_q, up_q,
                       out_q, reinterpret_cast<half8*>(out16), gelu_lut);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "geglu16 launch");
    return G4A_OK;
}

extern "C" int g4a_plegate16(int n_rows, int d, const void* lin16, float lin_q, const float* ple, int ple_stride,
                             float out_q, void* out16, const float* gelu_lut, void* stream) {
    if (n_rows <= 0 || d <= 0 || d % 8 || ple_stride < d || ple_stride % 4 || (int64_t)n_rows * d > 0x7fffffff) {
        set_error("n_rows, d (a multiple of 8) positive, ple_stride >= d and a multiple of 4");
        return G4A_EINVAL;
    }
    if (!lin16 || !ple || !out16 || (((uintptr_t)lin16 | (uintptr_t)ple | (uintptr_t)out16) & 15)) {
        set_error("lin, ple and out must be non-NULL and 16-byte aligned");
        return G4A_EINVAL;
    }
    if (!(lin_q >= 0.0f) || !(out_q >= 0.0f)) {
        set_error("lin_q and out_q must be >= 0");
        return G4A_EINVAL;
    }
    const int n8 = n_rows * d / 8;
    hipLaunchKernelGGL(plegate16_kernel, dim3((n8 + 255) / 256), dim3(256), 0, (hipStream_t)stream, n8, d,
                       reinterpret_cast<const half8*>(lin16), lin_q, ple, ple_stride, out_q,
                       reinterpret_cast<half8*>(out16), gelu_lut);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "plegate16 launch");
    return G4A_OK;
}
