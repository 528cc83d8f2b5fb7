// The rest of one decode step around the attention block: the QAT linears after it
// (o_proj, the gate/up/down MLP, the int8 per-layer-embedding gate and projection, the
// 2-bit lm_head), the sandwich RMSNorms with their residual adds, GeGLU, the token and
// per-layer embedding rows, and the logit softcap + greedy argmax that keep the next token
// on the device (gemma4_150/reference.py:132-207; the runner's kernels 69, 73-77, 33 and
// the argmax at runner.py:373-470).
//
// Every kernel here is bound by HBM (weight rows read once) or is a single-row vector op;
// none of them carries MFMA-shaped work.
#include <math.h>

#include "common.hpp"

namespace g4a {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- quantised GEMV
// out[o] = srq(scale[o] * sum_i (q[o][i] - zp) * srq(x[i], in_q), out_q)
// (reference.py:99-104 _qlin, :106-114 _ilin_raw with the biased int8 codes of export.py:150-156,
// :202-206 lm_head). Rows are packed BITS-bit values, value i of a row at bit
// BITS*(i % (32/BITS)) of word i / (32/BITS) (the loader's and dq_f16's order); zp =
// 2^(BITS-1). BITS = 16: plain f16 rows (pl_model_proj), no zero point, no row scale.
// A wave splits into 64/LPR lane groups; a group owns RPW rows and walks their 16-byte
// chunks LPR at a time, so short rows (the 384-byte lm_head rows) keep every lane busy.
struct QgemvArgs {
    const float* x;
    const uint32_t* w;
    const float* scale;  // [n_out], NULL: 1
    float* out;
    int n_in, n_out, row_chunks;  // 16-byte chunks per row
    float in_q, out_q;
};

template <int BITS, int LPR, int RPW>
__global__ __launch_bounds__(256) void qgemv_kernel(QgemvArgs g) {
    constexpr int VPC = 128 / BITS;  // values per 16-byte chunk
    constexpr int VPW = 32 / BITS;   // values per word
    constexpr int NG = 64 / LPR;
    constexpr float ZP = BITS == 16 ? 0.0f : (float)(1 << (BITS - 1));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, grp = lane / LPR;
    const int row0 = ((blockIdx.x * 4 + wave) * NG + grp) * RPW;
    const int nch = g.row_chunks;
    // rows past n_out and chunks past a row read as zeros through the buffer ranges
    const rsrc_t rw = make_rsrc(g.w, (uint32_t)g.n_out * (uint32_t)nch * 16u);
    const rsrc_t rx = make_rsrc(g.x, (uint32_t)g.n_in * 4u);
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
    for (int c = sub; c < nch; c += LPR) {
        u32x4_t wv[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = row0 + r < g.n_out ? row0 + r : g.n_out;  // n_out: past the range
            wv[r] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rw, (row * nch + c) * 16, 0, kCpolNT));
        }
        float xv[VPC];
#pragma unroll
        for (int i = 0; i < VPC / 4; ++i) {
            const float4v v = bload_f32x4(rx, (c * VPC + 4 * i) * 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[4 * i + e] = srq(v[e], g.in_q);
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
#pragma unroll
            for (int j = 0; j < VPC; ++j) {
                const uint32_t word = wv[r][j / VPW];
                float wq;
                if constexpr (BITS == 16) {
                    const uint16_t h = (uint16_t)(word >> (16 * (j % 2)));
                    wq = (float)__builtin_bit_cast(half_t, h);
                } else {
                    wq = (float)((word >> (BITS * (j % VPW))) & ((1u << BITS) - 1u)) - ZP;
                }
                acc[r] = __builtin_fmaf(wq, xv[j], acc[r]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
#pragma unroll
        for (int off = LPR / 2; off > 0; off >>= 1) acc[r] += __shfl_xor(acc[r], off);
    }
    if (sub == 0) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            const int row = row0 + r;
            if (row < g.n_out) g.out[row] = srq((g.scale ? g.scale[row] : 1.0f) * acc[r], g.out_q);
        }
    }
}

// ---------------------------------------------------------------- RMSNorm family
// Row r of n values: y = x' / sqrt(mean(x'^2) + eps) * w, x' = x * pre; out = (res + y) * mult
// (reference.py:38-43 rms_norm, the sandwich adds of :150, :162, :170, :132-137 for the
// per-layer-embedding context). Optional second output out2 = srq(out, q2), or with f16_2
// f16(srq(f16(out), q2)) (the MLP input of :153-156), and sum2 = sum of out2 (the
// zero-point sum the q/k/v GEMV takes).
struct RmsArgs {
    const float* x;
    const float* w;
    const float* res;
    float* out;
    float* out2;
    float* sum2;
    int n;
    float pre, mult, eps, q2;
    int f16_2;
};

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();  // red may still be read from a previous reduction
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

__global__ __launch_bounds__(1024) void rms_kernel(RmsArgs a) {
    __shared__ float red[16];
    const int r = blockIdx.x, n = a.n;
    const float* x = a.x + (size_t)r * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = x[i] * a.pre;
        ss = __builtin_fmaf(v, v, ss);
    }
    const float d = sqrtf(block_sum(ss, red) / (float)n + a.eps);
    float s2 = 0.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float y = (x[i] * a.pre) / d;
        if (a.w) y *= a.w[i];
        if (a.res) y = a.res[(size_t)r * n + i] + y;
        y *= a.mult;
        a.out[(size_t)r * n + i] = y;
        if (a.out2) {
            const float y2 = a.f16_2 ? (float)(half_t)srq((float)(half_t)y, a.q2) : srq(y, a.q2);
            a.out2[(size_t)r * n + i] = y2;
            s2 += y2;
        }
    }
    if (a.sum2) {
        const float t = block_sum(s2, red);
        if (threadIdx.x == 0) a.sum2[r] = t;
    }
}

// ---------------------------------------------------------------- GeGLU
// out = srq(gelu_tanh(a) * b, q) (reference.py:33-35, :159, :167)
__device__ __forceinline__ float gelu_tanh(float v) {
    return 0.5f * v * (1.0f + tanhf(0.7978845608028654f * (v + 0.044715f * v * v * v)));
}

__global__ __launch_bounds__(256) void geglu_kernel(int n, const float* a, const float* b, float q, float* out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = srq(gelu_tanh(a[i]) * b[i], q);
}

// ---------------------------------------------------------------- embedding rows
// out[j] = mult * row_scale[tok * (n / group) + j / group] * (code_j - 2^(bits-1)) for the
// packed row tok of the table (reference.py:116-124 embed, 2-bit; :126-133 ple_table,
// 4-bit with one scale per layer slice). The token id is read on the device, so a step can
// start from the argmax of the previous one; an id past the table reads zeros.
__global__ __launch_bounds__(256) void embed_kernel(int bits, int n, const uint32_t* table, uint32_t table_bytes,
                                                    int row_words, const int32_t* tok, const float* row_scale,
                                                    uint32_t scale_bytes, int group, float mult, float* out) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    const int t = tok[0];
    const rsrc_t rt = make_rsrc(table, table_bytes);
    const rsrc_t rs = make_rsrc(row_scale, scale_bytes);
    const int vpw = 32 / bits;
    const int64_t wo = (int64_t)t * row_words + j / vpw;
    const uint32_t word = (t >= 0 && wo < (int64_t)(table_bytes / 4))
                              ? __builtin_amdgcn_raw_buffer_load_b32(rt, (int)(wo * 4), 0, 0)
                              : 0u;
    const uint32_t code = (word >> (bits * (j % vpw))) & ((1u << bits) - 1u);
    const int64_t so = (int64_t)t * (n / group) + j / group;
    const float sc = (t >= 0 && so < (int64_t)(scale_bytes / 4)) ? bload_f32(rs, (int)(so * 4)) : 0.0f;
    out[j] = mult * sc * ((float)code - (float)(1 << (bits - 1)));
}

// ---------------------------------------------------------------- softcap + argmax
// logits <- cap * tanh(logits / cap) (cap 0: unchanged), tok = the first index of the
// maximum (reference.py:207; numpy's argmax order). One workgroup.
__global__ __launch_bounds__(1024) void softcap_argmax_kernel(int n, float* logits, float cap, int32_t* tok) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float best = kNegInf;
    int bi = 0x7fffffff;
    for (int i = threadIdx.x; i < n; i += 1024) {
        float v = logits[i];
        if (cap != 0.0f) {
            v = cap * tanhf(v / cap);
            logits[i] = v;
        }
        if (v > best) {  // ascending i per thread: the first maximum stays
            best = v;
            bi = i;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int oi = __shfl_xor(bi, off);
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = best;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w)
            if (sv[w] > best || (sv[w] == best && si[w] < bi)) {
                best = sv[w];
                bi = si[w];
            }
        tok[0] = bi == 0x7fffffff ? 0 : bi;
    }
}

template <int BITS, int LPR, int RPW>
static hipError_t launch_qgemv(const QgemvArgs& g, hipStream_t s) {
    const int rows_per_wg = 4 * (64 / LPR) * RPW;
    hipLaunchKernelGGL((qgemv_kernel<BITS, LPR, RPW>), dim3((g.n_out + rows_per_wg - 1) / rows_per_wg), dim3(256), 0,
                       s, g);
    return hipGetLastError();
}

// lane-group width: the smallest power of two >= the chunks per row, at most 64
template <int BITS>
static hipError_t qgemv_dispatch(const QgemvArgs& g, hipStream_t s) {
    if (g.row_chunks <= 16) return launch_qgemv<BITS, 16, 2>(g, s);
    if (g.row_chunks <= 32) return launch_qgemv<BITS, 32, 2>(g, s);
    return launch_qgemv<BITS, 64, 2>(g, s);
}

static int qgemv_impl(int bits, int n_in, int n_out, const float* x, float in_q, const uint32_t* w,
                      const float* scale, float out_q, float* out, void* stream) {
    if (bits != 2 && bits != 4 && bits != 8 && bits != 16) {
        set_error("bits %d not supported (2, 4, 8, or 16 for f16 rows)", bits);
        return G4A_EUNSUPPORTED;
    }
    const int vpc = 128 / bits;
    if (n_in <= 0 || n_out <= 0 || n_in % vpc) {
        set_error("n_in (%d) must be a positive multiple of %d and n_out (%d) positive", n_in, vpc, n_out);
        return G4A_EINVAL;
    }
    const int64_t row_bytes = (int64_t)n_in * bits / 8;
    if ((int64_t)(n_out + 512) * row_bytes > 0x7fffffff || n_in > (1 << 24)) {
        set_error("weights beyond 32-bit buffer offsets");
        return G4A_EINVAL;
    }
    if (!x || !w || !out || (bits != 16 && !scale)) {
        set_error("x, w, out (and scale for quantised rows) must be non-NULL");
        return G4A_EINVAL;
    }
    if (((uintptr_t)x | (uintptr_t)w) & 15) {
        set_error("x and w must be 16-byte aligned");
        return G4A_EINVAL;
    }
    if (!(in_q >= 0.0f) || !(out_q >= 0.0f)) {
        set_error("in_q/out_q must be >= 0");
        return G4A_EINVAL;
    }
    QgemvArgs g;
    g.x = x;
    g.w = w;
    g.scale = bits == 16 ? nullptr : scale;
    g.out = out;
    g.n_in = n_in;
    g.n_out = n_out;
    g.row_chunks = (int)(row_bytes / 16);
    g.in_q = in_q;
    g.out_q = out_q;
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = bits == 2   ? qgemv_dispatch<2>(g, s)
                   : bits == 4 ? qgemv_dispatch<4>(g, s)
                   : bits == 8 ? qgemv_dispatch<8>(g, s)
                               : qgemv_dispatch<16>(g, s);
    if (e != hipSuccess) return hip_error(e, "qgemv launch");
    return G4A_OK;
}

}  // namespace g4a

using namespace g4a;

extern "C" int g4a_qgemv(int bits, int n_in, int n_out, const float* x, float in_q, const uint32_t* w_bits,
                         const float* w_scale, float out_q, float* out, void* stream) {
    if (bits == 16) {
        set_error("bits 16 is g4a_gemv_f16");
        return G4A_EUNSUPPORTED;
    }
    return qgemv_impl(bits, n_in, n_out, x, in_q, w_bits, w_scale, out_q, out, stream);
}

extern "C" int g4a_gemv_f16(int n_in, int n_out, const float* x, const void* w_f16, float* out, void* stream) {
    return qgemv_impl(16, n_in, n_out, x, 0.0f, (const uint32_t*)w_f16, nullptr, 0.0f, out, stream);
}

extern "C" int g4a_rms_norm(int n_rows, int n, const float* x, float pre, const float* w, const float* res,
                            float mult, float eps, float* out, float q2, int f16_2, float* out2, float* sum2,
                            void* stream) {
    if (n_rows <= 0 || n <= 0 || n_rows > 65535) {
        set_error("n_rows (%d) must be in [1, 65535] and n (%d) positive", n_rows, n);
        return G4A_EINVAL;
    }
    if (!x || !out || (sum2 && !out2)) {
        set_error("x and out (and out2 when sum2 is given) must be non-NULL");
        return G4A_EINVAL;
    }
    if (!(eps >= 0.0f) || !(q2 >= 0.0f)) {
        set_error("eps and q2 must be >= 0");
        return G4A_EINVAL;
    }
    RmsArgs a;
    a.x = x;
    a.w = w;
    a.res = res;
    a.out = out;
    a.out2 = out2;
    a.sum2 = sum2;
    a.n = n;
    a.pre = pre;
    a.mult = mult;
    a.eps = eps;
    a.q2 = q2;
    a.f16_2 = f16_2 != 0;
    const int threads = n >= 4096 ? 1024 : n >= 1024 ? 512 : 256;
    hipLaunchKernelGGL(rms_kernel, dim3(n_rows), dim3(threads), 0, (hipStream_t)stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "rms_norm launch");
    return G4A_OK;
}

extern "C" int g4a_geglu(int n, const float* a, const float* b, float out_q, float* out, void* stream) {
    if (n <= 0 || !a || !b || !out || !(out_q >= 0.0f)) {
        set_error("n must be positive, a, b, out non-NULL and out_q >= 0");
        return G4A_EINVAL;
    }
    hipLaunchKernelGGL(geglu_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, n, a, b, out_q, out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "geglu launch");
    return G4A_OK;
}

extern "C" int g4a_embed(int bits, int n, const void* table, int64_t n_rows, const int32_t* tok,
                         const float* row_scale, int group, float mult, float* out, void* stream) {
    if (bits != 2 && bits != 4 && bits != 8) {
        set_error("bits %d not supported (2, 4 or 8)", bits);
        return G4A_EUNSUPPORTED;
    }
    if (n <= 0 || n % (32 / bits) || group <= 0 || n % group || n_rows <= 0) {
        set_error("n (%d) must be a positive multiple of %d and of group (%d), n_rows positive", n, 32 / bits, group);
        return G4A_EINVAL;
    }
    const int row_words = n / (32 / bits);
    if (n_rows * row_words * 4 > 0x7fffffff || n_rows * (n / group) * 4 > 0x7fffffff) {
        set_error("table beyond 32-bit buffer offsets");
        return G4A_EINVAL;
    }
    if (!table || !tok || !row_scale || !out) {
        set_error("table, tok, row_scale and out must be non-NULL");
        return G4A_EINVAL;
    }
    hipLaunchKernelGGL(embed_kernel, dim3((n + 255) / 256), dim3(256), 0, (hipStream_t)stream, bits, n,
                       (const uint32_t*)table, (uint32_t)(n_rows * row_words * 4), row_words, tok, row_scale,
                       (uint32_t)(n_rows * (n / group) * 4), group, mult, out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "embed launch");
    return G4A_OK;
}

extern "C" int g4a_softcap_argmax(int n, float* logits, float cap, int32_t* tok, void* stream) {
    if (n <= 0 || !logits || !tok || !(cap >= 0.0f)) {
        set_error("n must be positive, logits and tok non-NULL, cap >= 0");
        return G4A_EINVAL;
    }
    hipLaunchKernelGGL(softcap_argmax_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, n, logits, cap, tok);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "softcap_argmax launch");
    return G4A_OK;
}
