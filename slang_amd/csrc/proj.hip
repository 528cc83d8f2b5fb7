// The q/k/v producer in front of the attention path, for gfx950: QAT-weight projections.
//
// Reference semantics:
//  * dq_f16 (gemma4_150/kernels_dsl.py:2101-2138): packed rows, value i of a row at bit
//    8*(i / (8/BITS)) + BITS*(i % (8/BITS)) of the row's bytes, w = f16(s_row * (q - 2^(BITS-1))).
//  * qkv_70 (kernels_dsl.py:1384-1480): decode GEMVs of q, k and v over one input a, 4-bit
//    rows, out[o] = srq(scale[o] * (sum_i q[o][i] a[i] - 8 sum_a), out_scale) with the zero
//    point folded into the input sum; one dispatch partitioned over the three matrices.
//  * prefill (prefill_gpu.py:327-342): srqh_b (a -> f16(srq(a, s)), kernels_dsl.py:233-242),
//    dq_f16, gemm_tiled (f32 accumulation, f16 result, :34-136), srq_b on the q path (:246-255).
//
// MI355X design (not the reference's):
//  * Decode reads the 4-bit rows straight from HBM (the bytes QAT saves are the bytes decode
//    pays for). A lane owns 16-byte chunks of a row (32 values) and keeps the matching 32
//    inputs in registers for every row it visits; values come out of the packed words with
//    byte masks and v_cvt_f32_ubyte*, and a row is one wave-wide DPP/permlane sum.
//  * Prefill is MFMA work. Weights are static, and 288 GB of HBM holds every layer's f16
//    weights many times over, so dequantisation is its own pass (g4a_dequant, run at load
//    or per call as the reference does) rather than VALU work repeated inside every GEMM
//    tile. The GEMM is a K-major ("TN") f16 MFMA GEMM, 32x32x16 tiles, computed transposed
//    (D^T = W . A^T) so each lane holds 4 consecutive output columns of one token and stores
//    them in one instruction; srqh_b is fused into the A staging and srq_b into the store.
#include <stdio.h>

#include "common.hpp"

namespace g4a {

typedef float float16v __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

static __device__ __forceinline__ float16v proj_mfma32(half8 a, half8 b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------- dequantisation
// One thread per 16 bytes of packed row (4 words): 128/BITS values, f16(s * (q - zp)).
template <int BITS>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ bits,
                                                      const float* __restrict__ scale,
                                                      half_t* __restrict__ out, int n_in,
                                                      int n_quads) {
    constexpr int VPQ = 128 / BITS;  // values per 16 bytes
    constexpr uint32_t MASK = (1u << BITS) - 1;
    const float zp = (float)(1 << (BITS - 1));
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n_quads) return;
    const int qpr = n_in / VPQ;  // quads per row
    const int o = i / qpr;
    const u32x4 w = *reinterpret_cast<const u32x4*>(bits + 4 * (size_t)i);
    const float s = scale[o];
    half_t* dst = out + (size_t)i * VPQ;
#pragma unroll
    for (int g = 0; g < VPQ / 8; ++g) {  // 8 values per 16-byte store
        half8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int v = 8 * g + j;                      // value within the 16 bytes
            const int bit = 32 * (v / (32 / BITS)) + 8 * ((v % (32 / BITS)) / (8 / BITS)) +
                            BITS * (v % (8 / BITS));      // word, byte, then low bits first
            const uint32_t q = (w[bit / 32] >> (bit % 32)) & MASK;
            h[j] = (half_t)(s * ((float)q - zp));
        }
        *reinterpret_cast<half8*>(dst + 8 * g) = h;
    }
}

// ---------------------------------------------------------------- decode q/k/v GEMV
struct GemvArgs {
    const float* a;
    const float* sum_a;
    const uint32_t* bits[3];
    const float* scales;  // [q_dim + 2 kv_dim]: q rows, then k, then v
    float* out[3];
    float out_scale[3];
    int hidden, q_dim, kv_dim;
};

// NJ chunks of 32 values per lane (hidden <= 2048 * NJ); RPW rows per wave, 4 waves.
template <int NJ, int RPW>
__global__ __launch_bounds__(256) void qkv_gemv_kernel(GemvArgs g) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * 4 + wave) * RPW;  // over [q rows | k rows | v rows]
    const int mat = row0 < g.q_dim ? 0 : row0 < g.q_dim + g.kv_dim ? 1 : 2;
    const int r0 = row0 - (mat == 0 ? 0 : mat == 1 ? g.q_dim : g.q_dim + g.kv_dim);
    const int nrows = mat == 0 ? g.q_dim : g.kv_dim;
    const int row_bytes = g.hidden / 2;
    // every operand load first: the input chunks, the packed rows, the scales and the sum
    const rsrc_t ra = make_rsrc(g.a, (uint32_t)g.hidden * 4);
    const rsrc_t rw = make_rsrc(g.bits[mat], (uint32_t)nrows * row_bytes);
    float av[NJ][32];
    u32x4 wv[RPW][NJ];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = lane + 64 * j;  // chunk of the row; past the row end reads zeros
            const int off = c < row_bytes / 16 ? (r0 + r) * row_bytes + 16 * c : 0x7fffffff;
            wv[r][j] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, 0);
        }
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int q4 = 0; q4 < 8; ++q4) {
            const float4v v = bload_f32x4(ra, 128 * (lane + 64 * j) + 16 * q4);
#pragma unroll
            for (int i = 0; i < 4; ++i) av[j][4 * q4 + i] = v[i];
        }
    const float sa = g.sum_a[0];
    float sc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) sc[r] = g.scales[(row0 + r)];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t lo = wv[r][j][k] & 0x0F0F0F0Fu, hi = (wv[r][j][k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                for (int b = 0; b < 4; ++b) {  // byte b: low nibble = value 2b, high = 2b + 1
                    acc = __builtin_fmaf((float)((lo >> (8 * b)) & 0xFFu), av[j][8 * k + 2 * b], acc);
                    acc = __builtin_fmaf((float)((hi >> (8 * b)) & 0xFFu), av[j][8 * k + 2 * b + 1], acc);
                }
            }
        acc = wave_sum(acc);
        if (lane == 0) g.out[mat][r0 + r] = srq(sc[r] * (acc - 8.0f * sa), g.out_scale[mat]);
    }
}

// ---------------------------------------------------------------- prefill projection GEMM
struct GemmArgs {
    const float* a;   // [M][K] f32
    const half_t* w;  // [N][K] f16
    void* out;        // [M][N] f16, or f32 with out_f32
    int M, N, K;
    float a_in_q, out_q;
};

// LDS tile rows are 32 halves (64 B, 4 chunks of 16 B); chunk c of row r sits at position
// c ^ ((r >> 2) & 3), so the 16 rows one 16-lane quarter of a b128 operand read touches,
// and the 8 rows x 2 chunks of a staging store, fall in 16 distinct bank groups.
__device__ __forceinline__ int gswz(int r, int c) { return r * 64 + 16 * (c ^ ((r >> 2) & 3)); }

template <bool OUT_F32>
__global__ __launch_bounds__(256) void proj_gemm_kernel(GemmArgs g) {
    constexpr int BM = 128, BN = 128, BK = 32, TILE = 128 * 64;  // bytes per LDS operand tile
    __shared__ __attribute__((aligned(1024))) char lds[2 * 2 * TILE];  // [buffer][W, A]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int l32 = lane & 31, h = lane >> 5;

    // staging: thread t moves 16 k-values of row t/2 (k half t%2) of both operands
    const int sr = tid >> 1, skh = tid & 1;
    const rsrc_t ra = make_rsrc(g.a, (uint32_t)g.M * g.K * 4);  // rows >= M read as zeros
    const rsrc_t rw = make_rsrc(g.w, (uint32_t)g.N * g.K * 2);
    const int a_off = (m0 + sr) * g.K * 4 + 64 * skh;
    const int w_off = (n0 + sr) * g.K * 2 + 32 * skh;
    float4v ast[4];
    u32x4 wst[2];
    auto stage_load = [&](int k0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) ast[i] = bload_f32x4(ra, a_off + 4 * k0 + 16 * i);
#pragma unroll
        for (int i = 0; i < 2; ++i) wst[i] = __builtin_amdgcn_raw_buffer_load_b128(rw, w_off + 2 * k0 + 16 * i, 0, 0);
    };
    auto stage_store = [&](int buf) {
        char* wl = lds + buf * 2 * TILE;
        char* al = wl + TILE;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            half8 hv;
#pragma unroll
            for (int j = 0; j < 4; ++j) {  // srqh_b: f16(srq(a, a_in_q))
                hv[j] = (half_t)srq(ast[2 * i][j], g.a_in_q);
                hv[4 + j] = (half_t)srq(ast[2 * i + 1][j], g.a_in_q);
            }
            *reinterpret_cast<half8*>(al + gswz(sr, 2 * skh + i)) = hv;
            *reinterpret_cast<u32x4*>(wl + gswz(sr, 2 * skh + i)) = wst[i];
        }
    };

    float16v acc[2][2] = {{float16v{}, float16v{}}, {float16v{}, float16v{}}};
    const int nk = g.K / BK;
    stage_load(0);
    stage_store(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        if (kt + 1 < nk) stage_load((kt + 1) * BK);
        const char* wl = lds + (kt & 1) * 2 * TILE;
        const char* al = wl + TILE;
#pragma unroll
        for (int s = 0; s < 2; ++s) {  // 16-value k-steps: lane (l32, h) holds k 8h .. 8h+7
            half8 wo[2], ao[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                wo[b] = *reinterpret_cast<const half8*>(wl + gswz(64 * wn + 32 * b + l32, 2 * s + h));
                ao[b] = *reinterpret_cast<const half8*>(al + gswz(64 * wm + 32 * b + l32, 2 * s + h));
            }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) acc[nb][mb] = proj_mfma32(wo[nb], ao[mb], acc[nb][mb]);
        }
        if (kt + 1 < nk) stage_store((kt + 1) & 1);
        __syncthreads();
    }

    // D^T[n][m]: acc[r] is column n = 8(r/4) + 4h + r%4, token m = l32 of the 32x32 block;
    // the GEMM result rounds to f16 (gemm_tiled), the q path then applies srq_b
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const int m = m0 + 64 * wm + 32 * mb + l32;
        if (m >= g.M) continue;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + 64 * wn + 32 * nb + 8 * q + 4 * h;
                float4v v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = (float)(half_t)acc[nb][mb][4 * q + i];
                if (OUT_F32)
                    store4(reinterpret_cast<float*>(g.out) + (size_t)m * g.N + n, srq4(v, g.out_q));
                else
                    store4(reinterpret_cast<half_t*>(g.out) + (size_t)m * g.N + n, v);
            }
    }
}

}  // namespace g4a

using namespace g4a;

extern "C" int g4a_dequant(int bits, int n_in, int n_out, const uint32_t* w_bits, const float* w_scale,
                           void* out_f16, void* stream) {
    if (bits != 2 && bits != 4 && bits != 8) {
        set_error("bits %d not supported (2, 4 or 8)", bits);
        return G4A_EUNSUPPORTED;
    }
    if (n_in <= 0 || n_out <= 0 || n_in % (128 / bits) || (int64_t)n_in * n_out > 0x7fffffff) {
        set_error("n_in (%d) must be a positive multiple of %d and n_in*n_out < 2^31 (n_out %d)", n_in,
                  128 / bits, n_out);
        return G4A_EINVAL;
    }
    if (!w_bits || !w_scale || !out_f16) {
        set_error("w_bits, w_scale and out must be non-NULL");
        return G4A_EINVAL;
    }
    if (((uintptr_t)w_bits | (uintptr_t)out_f16) & 15) {
        set_error("w_bits and out must be 16-byte aligned");
        return G4A_EINVAL;
    }
    const int n_quads = (int)((int64_t)n_out * n_in / (128 / bits));
    const dim3 grid((n_quads + 255) / 256);
    half_t* o = reinterpret_cast<half_t*>(out_f16);
    if (bits == 2) hipLaunchKernelGGL(dequant_kernel<2>, grid, dim3(256), 0, (hipStream_t)stream, w_bits, w_scale, o, n_in, n_quads);
    if (bits == 4) hipLaunchKernelGGL(dequant_kernel<4>, grid, dim3(256), 0, (hipStream_t)stream, w_bits, w_scale, o, n_in, n_quads);
    if (bits == 8) hipLaunchKernelGGL(dequant_kernel<8>, grid, dim3(256), 0, (hipStream_t)stream, w_bits, w_scale, o, n_in, n_quads);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "dequant launch");
    return G4A_OK;
}

extern "C" int g4a_qkv_gemv(int hidden, int q_dim, int kv_dim, const float* a, const float* sum_a,
                            const uint32_t* q_bits, const uint32_t* k_bits, const uint32_t* v_bits,
                            const float* scales, float q_out, float k_out, float v_out, float* out_q,
                            float* out_k, float* out_v, void* stream) {
    if (hidden <= 0 || hidden % 32 || hidden > 4096) {
        set_error("hidden (%d) must be a positive multiple of 32, at most 4096", hidden);
        return G4A_EINVAL;
    }
    if (q_dim <= 0 || q_dim % 8 || kv_dim < 0 || kv_dim % 8) {
        set_error("q_dim (%d) must be a positive and kv_dim (%d) a non-negative multiple of 8", q_dim, kv_dim);
        return G4A_EINVAL;
    }
    if (!a || !sum_a || !q_bits || !scales || !out_q || (kv_dim && (!k_bits || !v_bits || !out_k || !out_v))) {
        set_error("a, sum_a, q_bits, scales, out_q (and with kv_dim > 0 k_bits, v_bits, out_k, out_v) "
                  "must be non-NULL");
        return G4A_EINVAL;
    }
    if (((uintptr_t)a | (uintptr_t)q_bits | (uintptr_t)k_bits | (uintptr_t)v_bits) & 15) {
        set_error("a and the packed weights must be 16-byte aligned");
        return G4A_EINVAL;
    }
    if ((int64_t)q_dim * hidden / 2 > 0x7fffffff) {
        set_error("q rows beyond 32-bit buffer offsets");
        return G4A_EINVAL;
    }
    if (!(q_out >= 0.0f) || !(k_out >= 0.0f) || !(v_out >= 0.0f)) {
        set_error("q_out/k_out/v_out must be >= 0");
        return G4A_EINVAL;
    }
    GemvArgs g;
    g.a = a;
    g.sum_a = sum_a;
    g.bits[0] = q_bits;
    g.bits[1] = k_bits;
    g.bits[2] = v_bits;
    g.scales = scales;
    g.out[0] = out_q;
    g.out[1] = out_k;
    g.out[2] = out_v;
    g.out_scale[0] = q_out;
    g.out_scale[1] = k_out;
    g.out_scale[2] = v_out;
    g.hidden = hidden;
    g.q_dim = q_dim;
    g.kv_dim = kv_dim;
    const int total = q_dim + 2 * kv_dim;  // rows; 2 per wave, 8 per workgroup
    const dim3 grid(total / 8);
    if (hidden <= 2048)
        hipLaunchKernelGGL((qkv_gemv_kernel<1, 2>), grid, dim3(256), 0, (hipStream_t)stream, g);
    else
        hipLaunchKernelGGL((qkv_gemv_kernel<2, 2>), grid, dim3(256), 0, (hipStream_t)stream, g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "qkv_gemv launch");
    return G4A_OK;
}

extern "C" int g4a_proj_gemm(int M, int N, int K, const float* a, float a_in_q, const void* w_f16,
                             void* out, int out_f32, float out_q, void* stream) {
    if (M <= 0 || N <= 0 || K <= 0 || N % 128 || K % 32) {
        set_error("M (%d) must be positive, N (%d) a multiple of 128 and K (%d) of 32", M, N, K);
        return G4A_EINVAL;
    }
    if ((int64_t)(M + 127) * K * 4 > 0x7fffffff || (int64_t)N * K * 2 > 0x7fffffff ||
        (int64_t)M * N > 0x7fffffff) {
        set_error("operands beyond 32-bit buffer offsets");
        return G4A_EINVAL;
    }
    if (!a || !w_f16 || !out) {
        set_error("a, w and out must be non-NULL");
        return G4A_EINVAL;
    }
    if (((uintptr_t)a | (uintptr_t)w_f16 | (uintptr_t)out) & 15) {
        set_error("a, w and out must be 16-byte aligned");
        return G4A_EINVAL;
    }
    if (!(a_in_q >= 0.0f) || !(out_q >= 0.0f)) {
        set_error("a_in_q/out_q must be >= 0");
        return G4A_EINVAL;
    }
    GemmArgs g;
    g.a = a;
    g.w = reinterpret_cast<const half_t*>(w_f16);
    g.out = out;
    g.M = M;
    g.N = N;
    g.K = K;
    g.a_in_q = a_in_q;
    g.out_q = out_q;
    const dim3 grid(N / 128, (M + 127) / 128);
    if (out_f32)
        hipLaunchKernelGGL(proj_gemm_kernel<true>, grid, dim3(256), 0, (hipStream_t)stream, g);
    else
        hipLaunchKernelGGL(proj_gemm_kernel<false>, grid, dim3(256), 0, (hipStream_t)stream, g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "proj_gemm launch");
    return G4A_OK;
}
