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
// (reference.py:96-101 _qlin, :103-111 _ilin_raw with the biased int8 codes of
// export.py:150-156, :200-206 lm_head). Rows are packed BITS-bit values, value i of a row at
// bit BITS*(i % (32/BITS)) of word i / (32/BITS) (the loader's and dq_f16's order); zp =
// 2^(BITS-1). BITS = 16: plain f16 rows (pl_model_proj), no zero point, no row scale.
// A workgroup splits into 256/T row groups of T threads (T = 16 .. 256, sized to the row);
// a group owns RPW rows and walks their 16-byte chunks T at a time, so short rows (the
// 384-byte lm_head rows) keep most threads busy and each chunk of x serves RPW rows.
// Codes are decoded through byte lanes and the zero point comes out of the sum of x.
// Epilogues (EPI):
//   0  out = y
//   1  gate/up pair (gateup_74/95): y_b from the second matrix, out = srq(gelu(y) * y_b, epi_q)
//   2  out = gelu(y) * mul[o] (plegate_76: the gate times the layer's per-layer input)
struct QgemvArgs {
    const float* x;
    const uint32_t* w;
    const float* scale;  // [n_out], NULL: 1
    float* out;
    int n_in, n_out, row_chunks;  // 16-byte chunks per row
    float in_q, out_q;
    const uint32_t* w2;  // EPI 1: the up rows, their scales and steps
    const float* scale2;
    float in_q2, out_q2, epi_q;
    const float* mul;  // EPI 2
    const float* lut;  // EPI 1, 2: the layer's GELU table of the out_q grid (gelu_srq), or NULL
    // norm prologue (pa != NULL, staged kernels only): x = res + rms(pa) * w1, stored to xout by
    // workgroup 0; z = rms(x) * w2 (w2 != NULL) or x; the GEMV input is f16 ? f16(srq(f16(z),
    // q2)) : srq(z, q2), stored to zout (if given) by workgroup 0 -- the rms_kernel arithmetic
    const float* pa;
    const float* pres;
    const float* pw1;
    const float* pw2;
    float* pxout;
    float* pzout;
    float pq2, peps, pmult;
    int pf16;
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

// a reduction buffer written once per kernel: no barrier before the write
__device__ __forceinline__ float block_sum_once(float v, float* red) {
    v = wave_sum(v);
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// gelu with the tanh approximation in its exp2 form (gelu_tanh16, the batched prefill's): the
// libm tanhf form cost the decode step 1.665 -> 1.642 ms/token in the GEMV epilogues
__device__ __forceinline__ float gelu_tanh(float v) { return gelu_tanh16(v); }

// sum over the LPR lanes of a lane group (16, 32 or 64), every lane of the group gets it
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
    v = row16_sum(v);
    if constexpr (LPR >= 32) v = add16(v);
    if constexpr (LPR == 64) v = add32(v);
    return v;
}
// group_sum in int32 (the integer dot products' partial sums): exact at any magnitude
template <int N>
__device__ __forceinline__ int dpp_ror_i(int x) {
    return __builtin_amdgcn_update_dpp(0, x, 0x120 + N, 0xF, 0xF, false);
}
template <int LPR>
__device__ __forceinline__ int group_sum_i(int v) {
    v += dpp_ror_i<8>(v);
    v += dpp_ror_i<4>(v);
    v += dpp_ror_i<2>(v);
    v += dpp_ror_i<1>(v);
    if constexpr (LPR >= 32) {
        const auto p = __builtin_amdgcn_permlane16_swap((unsigned)v, (unsigned)v, false, false);
        v = (int)p[0] + (int)p[1];
    }
    if constexpr (LPR == 64) {
        const auto p = __builtin_amdgcn_permlane32_swap((unsigned)v, (unsigned)v, false, false);
        v = (int)p[0] + (int)p[1];
    }
    return v;
}

// acc += sum_j q_j * x[j] over the VPC values of one 16-byte chunk, x from LDS in the
// interleaved layout below. Codes go through byte lanes (v_cvt_f32_ubyteN after one mask):
// the zero point is taken out once per row from the sum of x, as qkv_70 does.
template <int BITS>
__device__ __forceinline__ float chunk_dot(u32x4_t w, const float4v* xq, int stride, float acc) {
    constexpr int VPC = 128 / BITS;
    float v[VPC];  // the chunk's codes (f16 values for BITS 16) in row order
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // word k holds values VPC/4*k ..
        const uint32_t u = w[k];
        float* vk = v + (VPC / 4) * k;
        if constexpr (BITS == 16) {
            vk[0] = (float)__builtin_bit_cast(half_t, (uint16_t)(u & 0xFFFFu));
            vk[1] = (float)__builtin_bit_cast(half_t, (uint16_t)(u >> 16));
        } else if constexpr (BITS == 8) {
#pragma unroll
            for (int b = 0; b < 4; ++b) vk[b] = (float)((u >> (8 * b)) & 0xFFu);
        } else {
            constexpr int PB = 8 / BITS;  // values per byte
            constexpr uint32_t M = BITS == 4 ? 0x0F0F0F0Fu : 0x03030303u;
#pragma unroll
            for (int f = 0; f < PB; ++f) {
                const uint32_t m = (u >> (BITS * f)) & M;  // value PB*b + f sits in byte b
#pragma unroll
                for (int b = 0; b < 4; ++b) vk[PB * b + f] = (float)((m >> (8 * b)) & 0xFFu);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < VPC / 4; ++e) {
        const float4v xv = xq[e * stride];
#pragma unroll
        for (int t = 0; t < 4; ++t) acc = __builtin_fmaf(v[4 * e + t], xv[t], acc);
    }
    return acc;
}

// The same sum in integers when x is on its quantisation grid (x = k * in_q, k in [-128, 127]):
// the codes times the int8 k with v_dot4_i32_i8, exact. 4-bit: the even and odd nibbles of
// word w come out as bytes (codes 0..15) and meet the k of the same values, staged per chunk
// as 8 dwords (dword 2w: values 8w, 8w+2, 8w+4, 8w+6; dword 2w+1: the odd ones) in two
// uint4 planes [2][nch]; the zero point is taken out afterwards as in chunk_dot. 2-bit: bit
// pair f of every byte of word w (mask after a shift by 2f) gives values 16w + 4b + f in
// byte b, against plane f of four [4][nch] (dword w of plane f: those values' k). 8-bit: the
// biased codes XOR 0x80 are the signed c - 128, against k in row order (one plane).
template <int BITS>
__device__ __forceinline__ int chunk_idot(u32x4_t w, const u32x4_t* xk, int stride, int acc) {
    if constexpr (BITS == 4) {
        const u32x4_t x0 = xk[0], x1 = xk[stride];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = w[k] & 0x0F0F0F0Fu, hi = (w[k] >> 4) & 0x0F0F0F0Fu;
            const uint32_t xe = k < 2 ? x0[2 * k] : x1[2 * k - 4], xo = k < 2 ? x0[2 * k + 1] : x1[2 * k - 3];
            acc = __builtin_amdgcn_sdot4((int)lo, (int)xe, acc, false);
            acc = __builtin_amdgcn_sdot4((int)hi, (int)xo, acc, false);
        }
    } else if constexpr (BITS == 2) {
#pragma unroll
        for (int f = 0; f < 4; ++f) {
            const u32x4_t xf = xk[f * stride];
#pragma unroll
            for (int k = 0; k < 4; ++k)
                acc = __builtin_amdgcn_sdot4((int)((w[k] >> (2 * f)) & 0x03030303u), (int)xf[k], acc, false);
        }
    } else {
        const u32x4_t x0 = xk[0];
#pragma unroll
        for (int k = 0; k < 4; ++k) acc = __builtin_amdgcn_sdot4((int)(w[k] ^ 0x80808080u), (int)x0[k], acc, false);
    }
    return acc;
}

template <int BITS, int T, int RPW, int EPI, int NT = 256, bool IDOT = false>
__global__ __launch_bounds__(NT) void qgemv_kernel(QgemvArgs g) {
    // T threads per row group (16..256, the chunks of a row spread over them), 256/T groups
    // per workgroup, RPW rows per group; groups wider than a wave reduce through LDS.
    // With several groups per workgroup (T <= 64), or a norm prologue (which needs all of x in
    // every workgroup anyway), x is quantised once per workgroup into LDS,
    // float4 i of chunk c at [i][c] (threads of a group read consecutive chunks: conflict-free),
    // one copy per matrix step; wider groups use each chunk of x in one thread only and load
    // it straight from memory.
    constexpr int VPC = 128 / BITS;  // values per 16-byte chunk
    static_assert(NT == 256 || (T <= 128 && NT <= 1024 && NT % 256 == 0), "workgroup shapes the launches use");
    constexpr int NGRP = NT / T;
    constexpr int NM = EPI == 1 ? 2 : 1;  // matrices
    // IDOT (2/4/8-bit rows, every in_q > 0; the host checks): x always staged, as its int8 grid
    // index k (also for groups wider than a wave), the dot products in integers (chunk_idot),
    // y = scale * (sum - zp * sum k) * in_q
    static_assert(!IDOT || BITS == 2 || BITS == 4 || BITS == 8, "integer dot products for 2-, 4- and 8-bit rows");
    constexpr float ZP = BITS == 16 || (IDOT && BITS == 8) ? 0.0f : (float)(1 << (BITS - 1));
    const bool stage = IDOT || T <= 64 || g.pa != nullptr;  // workgroup-uniform
    extern __shared__ float4v xs[];      // [NM][VPC/4][nch]
    __shared__ float red[T > 64 ? NT / 64 : 1][NM][RPW];
    __shared__ float xsum_part[16][NM];
    __shared__ float xsum_red[T > 64 ? NT / 64 : 1][NM];
    const int tid = threadIdx.x;
    const int sub = tid % T, grp = tid / T;
    const int row0 = (blockIdx.x * NGRP + grp) * RPW;
    const int nch = g.row_chunks, n_in = g.n_in;
    // rows past n_out read as zeros through the buffer range
    const uint32_t wbytes = (uint32_t)g.n_out * (uint32_t)nch * 16u;
    const rsrc_t rw[2] = {make_rsrc(g.w, wbytes), make_rsrc(EPI == 1 ? g.w2 : g.w, wbytes)};
    u32x4_t wv[NM][RPW];
    auto load_w = [&](int c) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                // n_out: past the range (zeros, no traffic), also for a lane with no chunk c
                const int row = row0 + r < g.n_out && c < nch ? row0 + r : g.n_out;
                wv[m][r] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                           rw[m], (row * nch + c) * 16, 0, kCpolNT));
            }
    };
    // Load order. Loads return in issue order, so a wait for a value also waits for every
    // load issued before it: the operands of the prologue and of the staging of x go out
    // first, then the epilogue's per-row operands, then the first weight chunk, which stays
    // in flight while x is normed and staged. All of them are straight-line buffer loads (a
    // load under a per-lane or skippable condition leaves the compiler unsure how many loads
    // follow it, and it then waits for all of them).
    constexpr int PER = (2048 + NT - 1) / NT;  // prologue values a thread (n_in <= 2048)
    float av[PER], rv[PER], w1v[PER], w2v[PER];
    // staging batches of x loaded before the weights: all of them (x <= 16384 values) for
    // the 256-thread groups of the wide rows (the down projection: 12288 inputs are three
    // batches, each a round trip of its own when loaded after the weights), else the first
    constexpr int XB = T == 256 ? 4 : 1;
    float4v xv[XB][4];
    const rsrc_t rx = make_rsrc(g.x, (uint32_t)n_in * 4u);
    if (g.pa) {  // workgroup-uniform
        const uint32_t nb = (uint32_t)n_in * 4u;
        const rsrc_t ra = make_rsrc(g.pa, nb), rr = make_rsrc(g.pres, nb), r1 = make_rsrc(g.pw1, nb),
                     r2 = make_rsrc(g.pw2, g.pw2 ? nb : 0u);
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int o = 4 * (tid + NT * k);  // past n_in: zeros
            av[k] = bload_f32(ra, o);
            rv[k] = bload_f32(rr, o);
            w1v[k] = bload_f32(r1, o);
            w2v[k] = bload_f32(r2, o);
        }
    } else if (stage) {
#pragma unroll
        for (int b = 0; b < XB; ++b)
#pragma unroll
            for (int k = 0; k < 4; ++k) xv[b][k] = bload_f32x4(rx, 4 * (16 * NT * b + 4 * (tid + NT * k)));
    }
    // the epilogue's per-row operands (thread r of a group writes row r) come in with the
    // first weight chunk: loaded in the epilogue they cost a memory round trip after the dot
    // products (1.1 us of the gate/up GEMV's 7 us, timestamped)
    const bool erow = sub < RPW && row0 + sub < g.n_out;
    const int eo = 4 * (erow ? row0 + sub : g.n_out);  // past the range: zeros
    const uint32_t ob = (uint32_t)g.n_out * 4u;
    float esc[NM], emul = 0.0f;
    esc[0] = bload_f32(make_rsrc(g.scale, g.scale ? ob : 0u), eo);
    if constexpr (EPI == 1) esc[NM - 1] = bload_f32(make_rsrc(g.scale2, g.scale2 ? ob : 0u), eo);
    if constexpr (EPI == 2) emul = bload_f32(make_rsrc(g.mul, ob), eo);
    load_w(sub);
    __builtin_amdgcn_sched_barrier(0);  // no prologue arithmetic (and its waits) above the weight loads
    if (!g.scale || !erow) esc[0] = 1.0f;
    if constexpr (EPI == 1)
        if (!g.scale2 || !erow) esc[NM - 1] = 1.0f;
    float sx[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) sx[m] = 0.0f;
    float* xsf = reinterpret_cast<float*>(xs);
    auto stage_x = [&](int i, float v) {
        const int c = i / VPC, e = i % VPC;
        if constexpr (IDOT) {
            // byte of value e of chunk c: 4-bit dword 2(e/8) + (e&1), byte (e%8)/2, in plane dword/4
            int at;
            if constexpr (BITS == 4) {
                const int dw = 2 * (e >> 3) + (e & 1);
                at = ((dw >> 2) * nch + c) * 16 + (dw & 3) * 4 + ((e & 7) >> 1);
            } else if constexpr (BITS == 2) {  // plane e % 4, dword e / 16, byte (e % 16) / 4
                at = ((e & 3) * nch + c) * 16 + (e >> 4) * 4 + ((e & 15) >> 2);
            } else {
                at = c * 16 + e;
            }
            signed char* xsb = reinterpret_cast<signed char*>(xs);
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const float k = fminf(fmaxf(rintf(v / (m == 0 ? g.in_q : g.in_q2)), -128.0f), 127.0f);  // srq's index
                xsb[m * n_in + at] = (signed char)(int)k;
                sx[m] += k;
            }
            return;
        }
        const int at = ((e >> 2) * nch + c) * 4 + (e & 3);
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const float q = srq(v, m == 0 ? g.in_q : g.in_q2);
            xsf[m * n_in + at] = q;
            sx[m] += q;
        }
    };
    if (g.pa) {  // workgroup-uniform; n_in <= 2048
        __shared__ float pred[2][16];  // one buffer per reduction
#pragma unroll
        for (int k = 0; k < PER; ++k) {  // the loaded zeros past n_in, and the unit gains
            const bool ok = tid + NT * k < n_in;
            if (!ok) w1v[k] = 1.0f;
            if (!ok || !g.pw2) w2v[k] = 1.0f;
        }
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; ++k) ss = __builtin_fmaf(av[k], av[k], ss);
        const float d = sqrtf(block_sum_once(ss, pred[0]) / (float)n_in + g.peps);
        float ss2 = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = tid + NT * k;
            const float y = (rv[k] + av[k] / d * w1v[k]) * g.pmult;
            av[k] = y;
            if (i < n_in) {
                if (blockIdx.x == 0) g.pxout[i] = y;
                ss2 = __builtin_fmaf(y, y, ss2);
            }
        }
        const float d2 = g.pw2 ? sqrtf(block_sum_once(ss2, pred[1]) / (float)n_in + g.peps) : 1.0f;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = tid + NT * k;
            const float z = g.pw2 ? av[k] / d2 * w2v[k] : av[k];
            const float zq = g.pf16 ? (float)(half_t)srq((float)(half_t)pin(z), g.pq2) : srq(z, g.pq2);
            if (i < n_in) {
                if (blockIdx.x == 0 && g.pzout) g.pzout[i] = zq;
                stage_x(i, zq);
            }
        }
    } else if (stage) {
        // every load of x first, in batches of 16 NT values (4 float4 a thread), then the
        // staging: one L2 round trip per batch instead of one per element. The batches
        // loaded before the weights are staged outside the loop (inside it, the join with
        // the loop's own loads would make their waits cover the weights again).
        auto stage_batch = [&](int b0, const float4v (&xb)[4]) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int i = b0 + 4 * (tid + NT * k);
                if (i < n_in) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) stage_x(i + e, xb[k][e]);
                }
            }
        };
#pragma unroll
        for (int b = 0; b < XB; ++b)
            if (16 * NT * b < n_in) stage_batch(16 * NT * b, xv[b]);
        for (int b0 = 16 * NT * XB; b0 < n_in; b0 += 16 * NT) {
#pragma unroll
            for (int k = 0; k < 4; ++k) xv[0][k] = bload_f32x4(rx, 4 * (b0 + 4 * (tid + NT * k)));
            stage_batch(b0, xv[0]);
        }
    }
    float xtot[NM];  // staged: the sum of the whole quantised x, known after the barrier
    if (stage) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            const float t = wave_sum(sx[m]);
            if ((tid & 63) == 0) xsum_part[tid >> 6][m] = t;
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < NM; ++m) {
            xtot[m] = (xsum_part[0][m] + xsum_part[1][m]) + (xsum_part[2][m] + xsum_part[3][m]);
            if constexpr (NT >= 512)
                xtot[m] += (xsum_part[4][m] + xsum_part[5][m]) + (xsum_part[6][m] + xsum_part[7][m]);
            if constexpr (NT == 768)
                xtot[m] += (xsum_part[8][m] + xsum_part[9][m]) + (xsum_part[10][m] + xsum_part[11][m]);
            if constexpr (NT == 1024)
                xtot[m] += ((xsum_part[8][m] + xsum_part[9][m]) + (xsum_part[10][m] + xsum_part[11][m])) +
                           ((xsum_part[12][m] + xsum_part[13][m]) + (xsum_part[14][m] + xsum_part[15][m]));
            sx[m] = 0.0f;
        }
    }
    // IDOT sums stay int32 to the end (exact at any row length); the others are f32
    float acc[NM][RPW];
    int iacc[NM][RPW];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            acc[m][r] = 0.0f;
            iacc[m][r] = 0;
        }
    for (int c = sub; c < nch; c += T) {
        if (c != sub) load_w(c);
        if constexpr (IDOT) {
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const u32x4_t* xk = reinterpret_cast<const u32x4_t*>(reinterpret_cast<const signed char*>(xs) + m * n_in) + c;
#pragma unroll
                for (int r = 0; r < RPW; ++r) iacc[m][r] = chunk_idot<BITS>(wv[m][r], xk, nch, iacc[m][r]);
            }
        } else if (stage) {
#pragma unroll
            for (int m = 0; m < NM; ++m)
#pragma unroll
                for (int r = 0; r < RPW; ++r)
                    acc[m][r] = chunk_dot<BITS>(wv[m][r], xs + (size_t)m * (VPC / 4) * nch + c, nch, acc[m][r]);
        } else {
            float4v xr[VPC / 4];
#pragma unroll
            for (int e = 0; e < VPC / 4; ++e) xr[e] = bload_f32x4(rx, (c * VPC + 4 * e) * 4);
#pragma unroll
            for (int m = 0; m < NM; ++m) {
                const float q = m == 0 ? g.in_q : g.in_q2;
                float4v xq[VPC / 4];
#pragma unroll
                for (int e = 0; e < VPC / 4; ++e) {
                    xq[e] = srq4(xr[e], q);
                    sx[m] += (xq[e][0] + xq[e][1]) + (xq[e][2] + xq[e][3]);
                }
#pragma unroll
                for (int r = 0; r < RPW; ++r) acc[m][r] = chunk_dot<BITS>(wv[m][r], xq, 1, acc[m][r]);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < NM; ++m) {
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
            if constexpr (IDOT) iacc[m][r] = group_sum_i<T >= 64 ? 64 : T>(iacc[m][r]);
            else acc[m][r] = group_sum<T >= 64 ? 64 : T>(acc[m][r]);
        }
        sx[m] = group_sum<64>(sx[m]);  // direct loads only (0 when staged)
    }
    if constexpr (T > 64) {  // the group's waves through LDS (one group per 128/256 threads)
        const int wig = sub >> 6;  // wave in group
        const int slot = grp * (T / 64) + wig;  // the wave's index
        if ((tid & 63) == 0) {
#pragma unroll
            for (int m = 0; m < NM; ++m) {
#pragma unroll
                for (int r = 0; r < RPW; ++r) red[slot][m][r] = IDOT ? __builtin_bit_cast(float, iacc[m][r]) : acc[m][r];
                xsum_red[slot][m] = sx[m];
            }
        }
        __syncthreads();
#pragma unroll
        for (int m = 0; m < NM; ++m) {
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                if constexpr (IDOT) {
                    int t = 0;
#pragma unroll
                    for (int k = 0; k < T / 64; ++k) t += __builtin_bit_cast(int, red[grp * (T / 64) + k][m][r]);
                    iacc[m][r] = t;
                } else {
                    float t = 0.0f;
#pragma unroll
                    for (int k = 0; k < T / 64; ++k) t += red[grp * (T / 64) + k][m][r];
                    acc[m][r] = t;
                }
            }
            float t = 0.0f;
#pragma unroll
            for (int k = 0; k < T / 64; ++k) t += xsum_red[grp * (T / 64) + k][m];
            sx[m] = t;
        }
    }
    float zsx[NM];  // zero point times the sum of the quantised x (over the whole row)
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        zsx[m] = ZP * (stage ? xtot[m] : sx[m]);
    }
    // thread r of the group writes row r
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row0 + r;
        if (sub == r && row < g.n_out) {
            // IDOT: D = sum - zp * sum k, exact in int32 (zp * sum k is an integer, exact in f32
            // for the <= 4096 staged codes), rounded to f32 once, times the input step
            const float d0 = IDOT ? (float)(iacc[0][r] - (int)zsx[0]) * g.in_q : acc[0][r] - zsx[0];
            float y = srq(esc[0] * d0, g.out_q);
            if constexpr (EPI == 1) {
                const float d1 = IDOT ? (float)(iacc[NM - 1][r] - (int)zsx[NM - 1]) * g.in_q2 : acc[NM - 1][r] - zsx[NM - 1];
                const float yb = srq(esc[NM - 1] * d1, g.out_q2);
                y = srq(gelu_srq(y, g.out_q, g.lut) * yb, g.epi_q);
            } else if constexpr (EPI == 2) {
                y = gelu_srq(y, g.out_q, g.lut) * emul;
            }
            g.out[row] = y;
        }
    }
}

// ---------------------------------------------------------------- RMSNorm family
// Row r of n values: y = x' / sqrt(mean(x'^2) + eps) * w, x' = x * pre; out = (res + y) * mult
// (reference.py:38-43 rms_norm, the sandwich adds of :170, :183, :191, :133-139 for the
// per-layer-embedding context). Optional second output from out itself or, with w2, from
// the next norm z = rms(out) * w2 (the runner's cross-kernel fusions: oproj_73 ends with the
// pre-FFN norm, pleproj_77 with the next layer's input norm): out2 = srq(z, q2), or with
// f16_2 f16(srq(f16(z), q2)) (the MLP input of :176-178), and sum2 = sum of out2 (the
// zero-point sum the q/k/v GEMV takes).
struct RmsArgs {
    const float* x;
    const float* w;
    const float* res;
    const float* w2;
    float* out;
    float* out2;
    float* sum2;
    int n;
    float pre, mult, eps, q2;
    int f16_2;
};

// Thread t holds elements t + k*blockDim (k < PER) in registers: every operand is loaded
// once, up front, and the three sums cost only LDS round trips.
template <int PER>
__global__ __launch_bounds__(1024) void rms_kernel(RmsArgs a) {
    __shared__ float red[16];
    const int r = blockIdx.x, n = a.n, nt = blockDim.x;
    const float* x = a.x + (size_t)r * n;
    float* out = a.out + (size_t)r * n;
    float xv[PER], wv[PER], rv[PER], w2v[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = threadIdx.x + k * nt;
        const bool ok = i < n;
        xv[k] = ok ? x[i] * a.pre : 0.0f;
        wv[k] = ok && a.w ? a.w[i] : 1.0f;
        rv[k] = ok && a.res ? a.res[(size_t)r * n + i] : 0.0f;
        w2v[k] = ok && a.w2 ? a.w2[i] : 1.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) ss = __builtin_fmaf(xv[k], xv[k], ss);
    const float d = sqrtf(block_sum(ss, red) / (float)n + a.eps);
    float ss2 = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = threadIdx.x + k * nt;
        float y = xv[k] / d;
        if (a.w) y *= wv[k];
        y = (rv[k] + y) * a.mult;
        xv[k] = y;
        if (i < n) {
            out[i] = y;
            ss2 = __builtin_fmaf(y, y, ss2);
        }
    }
    if (!a.out2) return;
    const float d2 = a.w2 ? sqrtf(block_sum(ss2, red) / (float)n + a.eps) : 1.0f;
    float s2 = 0.0f;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
        const int i = threadIdx.x + k * nt;
        const float z = a.w2 ? xv[k] / d2 * w2v[k] : xv[k];
        const float y2 = a.f16_2 ? (float)(half_t)srq((float)(half_t)pin(z), a.q2) : srq(z, a.q2);
        if (i < n) {
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
__global__ __launch_bounds__(256) void geglu_kernel(int n, const float* a, const float* b, float q, float* out) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = srq(gelu_tanh(a[i]) * b[i], q);
}

// ---------------------------------------------------------------- embedding rows
// out[j] = mult * row_scale[tok * (n / group) + j / group] * (code_j - 2^(bits-1)) for the
// packed row tok of the table (reference.py:116-124 embed, 2-bit; :126-133 ple_table,
// 4-bit with one scale per layer slice). The token id is read on the device, so a step can
// start from the argmax of the previous one; an id past the table reads zeros. Grid row y
// gathers token tok[y] into out + y*n (embed_00 / plegather_01 over S tokens).
__global__ __launch_bounds__(256) void embed_kernel(int bits, int n, const uint32_t* table, uint32_t table_bytes,
                                                    int row_words, const int32_t* tok, const float* row_scale,
                                                    uint32_t scale_bytes, int group, float mult, float* out) {
    const int j = blockIdx.x * 256 + threadIdx.x;
    if (j >= n) return;
    const int t = tok[blockIdx.y];
    out += (size_t)blockIdx.y * n;
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
// maximum (reference.py:207; numpy's argmax order). Two stages as the runner's argmax1_34 /
// argmax2_35 (runner.py:501-505): workgroup b caps and scans [b*kArgChunk, (b+1)*kArgChunk)
// and leaves its (max, first index) in part[b]; one workgroup reduces the parts.
constexpr int kArgChunk = 4096;

__device__ __forceinline__ void argmax_step(float& best, int& bi, float v, int i) {
    if (v > best || (v == best && i < bi)) {
        best = v;
        bi = i;
    }
}

// the workgroup's (max, first index) into lane 0 of wave 0
__device__ __forceinline__ void block_argmax(float& best, int& bi, float* sv, int* si) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(best, off);
        const int oi = __shfl_xor(bi, off);
        argmax_step(best, bi, ov, oi);
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[wave] = best;
        si[wave] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0)
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w) argmax_step(best, bi, sv[w], si[w]);
}

__global__ __launch_bounds__(256) void softcap_part_kernel(int n, float* logits, float cap, float2* part) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int base = blockIdx.x * kArgChunk;
    float best = kNegInf;
    int bi = 0x7fffffff;
#pragma unroll 4
    for (int k = 0; k < kArgChunk / 1024; ++k) {
        const int i0 = base + 4 * (k * 256 + (int)threadIdx.x);  // 4 consecutive logits per thread
        if (i0 + 3 < n) {
            float4v v = *reinterpret_cast<const float4v*>(logits + i0);
            if (cap != 0.0f) {
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = cap * tanhf(v[e] / cap);
                *reinterpret_cast<float4v*>(logits + i0) = v;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) argmax_step(best, bi, v[e], i0 + e);
        } else {
            for (int e = 0; e < 4 && i0 + e < n; ++e) {
                float v = logits[i0 + e];
                if (cap != 0.0f) {
                    v = cap * tanhf(v / cap);
                    logits[i0 + e] = v;
                }
                argmax_step(best, bi, v, i0 + e);
            }
        }
    }
    block_argmax(best, bi, sv, si);
    if (threadIdx.x == 0) part[blockIdx.x] = make_float2(best, __builtin_bit_cast(float, bi));
}

__global__ __launch_bounds__(1024) void argmax_final_kernel(int n_part, const float2* part, int32_t* tok) {
    __shared__ float sv[16];
    __shared__ int si[16];
    float best = kNegInf;
    int bi = 0x7fffffff;
    for (int b = threadIdx.x; b < n_part; b += 1024) {
        const float2 p = part[b];
        argmax_step(best, bi, p.x, __builtin_bit_cast(int, p.y));
    }
    block_argmax(best, bi, sv, si);
    if (threadIdx.x == 0) tok[0] = bi == 0x7fffffff ? 0 : bi;  // no finite maximum: 0, as numpy
}

template <int BITS, int T, int RPW, int EPI, int NT = 256>
static hipError_t launch_qgemv(const QgemvArgs& g, hipStream_t s) {
    const int rows_per_wg = (NT / T) * RPW;
    const bool staged = T <= 64 || g.pa;
    const size_t lds = staged ? (size_t)(EPI == 1 ? 2 : 1) * g.n_in * sizeof(float) : 0;
    const dim3 grid((g.n_out + rows_per_wg - 1) / rows_per_wg);
    if constexpr (BITS == 2 || BITS == 4 || BITS == 8) {
        // integer dot products where x is on a grid (every in_q > 0; whole chunks): x staged as
        // its int8 grid index, also for the wide rows that otherwise read x straight from memory
        if (g.in_q > 0.0f && (EPI != 1 || g.in_q2 > 0.0f) && g.n_in % (128 / BITS) == 0) {
            const size_t lds_i = staged ? lds : (size_t)(EPI == 1 ? 2 : 1) * g.n_in;
            hipLaunchKernelGGL((qgemv_kernel<BITS, T, RPW, EPI, NT, true>), grid, dim3(NT), lds_i, s, g);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((qgemv_kernel<BITS, T, RPW, EPI, NT>), grid, dim3(NT), lds, s, g);
    return hipGetLastError();
}

// Threads per row group: the smallest of 16..256 covering a row's chunks, so one pass
// reads every row of the workgroup and all of them are in flight together (decode GEMVs
// are latency-bound: o_proj and down have only 1536 rows). Rows per group: 8 for the
// short 2-bit rows of the lm_head (x loaded once per 8 rows), 1 for rows of at most 16
// chunks (the per-layer-embedding projection: twice the workgroups, 1.737 -> 1.727 ms a
// decode step), 3 for rows of more than 128 chunks (the down projection: 512 workgroups
// of 256 threads, two a CU, each x chunk serving 3 rows: 1.549 -> 1.537 ms a step; 4 rows
// gained nothing, 8 were 20 % slower), else 2.
template <int BITS, int EPI>
static hipError_t qgemv_dispatch(const QgemvArgs& g, hipStream_t s) {
    const int c = g.row_chunks;
    if (c <= 16) return launch_qgemv<BITS, 16, 1, EPI>(g, s);
    if (c <= 32) {
        if (BITS == 2 && g.pa)  // the double-wide 2-bit gate/up with its norm prologue: 12288 rows
                                // at 48 a workgroup of 768 threads, one workgroup a CU
            return launch_qgemv<BITS, 32, 2, EPI, 768>(g, s);
        return BITS == 2 ? launch_qgemv<BITS, 32, 8, EPI>(g, s) : launch_qgemv<BITS, 32, 2, EPI>(g, s);
    }
    if (c <= 64)  // the norm prologue once per 768 threads: fewer workgroups read its operands
                  // (the gate/up GEMV at E2B shape: whole step 1.807 -> 1.769 ms/token with 512
                  // threads, 1.746 with 1024; 768 gives its 6144 rows one workgroup per CU:
                  // 1.583 -> 1.571 against 1024)
        return BITS >= 4 && g.pa ? launch_qgemv<BITS, 64, 2, EPI, 768>(g, s)
                                 : launch_qgemv<BITS, 64, 2, EPI>(g, s);
    if (c <= 128)  // with a prologue (the PLE gate): 512 threads, 4 elements of it a thread, one
                   // row a group (its 256 rows in 64 workgroups, not 32: 1.540 -> 1.523 ms a
                   // step; 128 workgroups of 256 threads gained nothing)
        return BITS >= 4 && g.pa ? launch_qgemv<BITS, 128, 1, EPI, 512>(g, s) : launch_qgemv<BITS, 128, 2, EPI>(g, s);
    return launch_qgemv<BITS, 256, 3, EPI>(g, s);
}

static int qgemv_check(int bits, int n_in, int n_out, const float* x, const uint32_t* w, const float* scale,
                       const float* out, float in_q, float out_q) {
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
    if ((int64_t)(n_out + 512) * row_bytes > 0x7fffffff) {
        set_error("weights beyond 32-bit buffer offsets");
        return G4A_EINVAL;
    }
    if (n_in > 16384) {  // x is staged in LDS, two copies for the gate/up pair
        set_error("n_in (%d) above 16384", n_in);
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
    return G4A_OK;
}

static int qgemv_run(int bits, int epi, QgemvArgs& g, void* stream) {
    g.row_chunks = (int)((int64_t)g.n_in * bits / 128);
    hipStream_t s = (hipStream_t)stream;
    hipError_t e = hipSuccess;
    switch (epi * 32 + bits) {
        case 0 * 32 + 2: e = qgemv_dispatch<2, 0>(g, s); break;
        case 0 * 32 + 4: e = qgemv_dispatch<4, 0>(g, s); break;
        case 0 * 32 + 8: e = qgemv_dispatch<8, 0>(g, s); break;
        case 0 * 32 + 16: e = qgemv_dispatch<16, 0>(g, s); break;
        case 1 * 32 + 2: e = qgemv_dispatch<2, 1>(g, s); break;
        case 1 * 32 + 4: e = qgemv_dispatch<4, 1>(g, s); break;
        case 1 * 32 + 8: e = qgemv_dispatch<8, 1>(g, s); break;
        case 2 * 32 + 2: e = qgemv_dispatch<2, 2>(g, s); break;
        case 2 * 32 + 4: e = qgemv_dispatch<4, 2>(g, s); break;
        case 2 * 32 + 8: e = qgemv_dispatch<8, 2>(g, s); break;
        default: set_error("no GEMV for %d-bit rows with epilogue %d", bits, epi); return G4A_EUNSUPPORTED;
    }
    if (e != hipSuccess) return hip_error(e, "qgemv launch");
    return G4A_OK;
}

// the norm prologue: checks and arguments (x is then unused)
static int norm_in_set(const g4a_norm_in* pro, int n_in, QgemvArgs& g) {
    if (!pro) return G4A_OK;
    if (!pro->a || !pro->res || !pro->w1 || !pro->x_out || n_in > 2048 || !(pro->q2 >= 0.0f) || !(pro->eps >= 0.0f)) {
        set_error("norm prologue: a, res, w1, x_out non-NULL, n_in <= 2048, q2 and eps >= 0");
        return G4A_EINVAL;
    }
    // workgroup 0 stores x and z while the others still read a, res and w1
    const size_t vb = (size_t)n_in * sizeof(float);
    for (const void* out : {(const void*)pro->x_out, (const void*)pro->z_out})
        if (overlaps(out, pro->a, vb) || overlaps(out, pro->res, vb) || overlaps(out, pro->w1, vb)) {
            set_error("norm prologue: x_out and z_out must not overlap a, res or w1");
            return G4A_EINVAL;
        }
    g.pa = pro->a;
    g.pres = pro->res;
    g.pw1 = pro->w1;
    g.pw2 = pro->w2;
    g.pxout = pro->x_out;
    g.pzout = pro->z_out;
    g.pq2 = pro->q2;
    g.peps = pro->eps;
    g.pf16 = pro->f16 != 0;
    g.pmult = pro->mult != 0.0f ? pro->mult : 1.0f;
    return G4A_OK;
}

static QgemvArgs qgemv_args(int n_in, int n_out, const float* x, float in_q, const uint32_t* w, const float* scale,
                            float out_q, float* out) {
    QgemvArgs g{};
    g.x = x;
    g.w = w;
    g.scale = scale;
    g.out = out;
    g.n_in = n_in;
    g.n_out = n_out;
    g.in_q = in_q;
    g.out_q = out_q;
    return g;
}

}  // namespace g4a

using namespace g4a;

extern "C" int g4a_qgemv(int bits, int n_in, int n_out, const float* x, float in_q, const uint32_t* w_bits,
                         const float* w_scale, float out_q, float* out, void* stream) {
    if (bits == 16) {
        set_error("bits 16 is g4a_gemv_f16");
        return G4A_EUNSUPPORTED;
    }
    const int rc = qgemv_check(bits, n_in, n_out, x, w_bits, w_scale, out, in_q, out_q);
    if (rc != G4A_OK) return rc;
    QgemvArgs g = qgemv_args(n_in, n_out, x, in_q, w_bits, w_scale, out_q, out);
    return qgemv_run(bits, 0, g, stream);
}

extern "C" int g4a_qgemv_geglu(int bits, int n_in, int n_out, const float* x, const uint32_t* gate_bits,
                               const float* gate_scale, float gate_in_q, float gate_out_q, const uint32_t* up_bits,
                               const float* up_scale, float up_in_q, float up_out_q, float out_q, float* out,
                               const g4a_norm_in* pro, const float* gelu_lut, void* stream) {
    if (pro && pro->a) x = pro->a;  // checked as the input; the prologue makes the real one
    if (bits == 16) {
        set_error("bits 16 not supported for the gate/up pair");
        return G4A_EUNSUPPORTED;
    }
    int rc = qgemv_check(bits, n_in, n_out, x, gate_bits, gate_scale, out, gate_in_q, gate_out_q);
    if (rc == G4A_OK) rc = qgemv_check(bits, n_in, n_out, x, up_bits, up_scale, out, up_in_q, up_out_q);
    if (rc != G4A_OK) return rc;
    if (!(out_q >= 0.0f)) {
        set_error("out_q must be >= 0");
        return G4A_EINVAL;
    }
    QgemvArgs g = qgemv_args(n_in, n_out, x, gate_in_q, gate_bits, gate_scale, gate_out_q, out);
    if ((rc = norm_in_set(pro, n_in, g)) != G4A_OK) return rc;
    g.w2 = up_bits;
    g.scale2 = up_scale;
    g.in_q2 = up_in_q;
    g.out_q2 = up_out_q;
    g.epi_q = out_q;
    g.lut = gelu_lut;
    return qgemv_run(bits, 1, g, stream);
}

extern "C" int g4a_qgemv_gelu_mul(int bits, int n_in, int n_out, const float* x, float in_q, const uint32_t* w_bits,
                                  const float* w_scale, float out_q, const float* mul, float* out,
                                  const g4a_norm_in* pro, const float* gelu_lut, void* stream) {
    if (pro && pro->a) x = pro->a;
    if (bits == 16) {
        set_error("bits 16 not supported with the gelu epilogue");
        return G4A_EUNSUPPORTED;
    }
    int rc = qgemv_check(bits, n_in, n_out, x, w_bits, w_scale, out, in_q, out_q);
    if (rc != G4A_OK) return rc;
    if (!mul) {
        set_error("mul must be non-NULL");
        return G4A_EINVAL;
    }
    QgemvArgs g = qgemv_args(n_in, n_out, x, in_q, w_bits, w_scale, out_q, out);
    if ((rc = norm_in_set(pro, n_in, g)) != G4A_OK) return rc;
    g.mul = mul;
    g.lut = gelu_lut;
    return qgemv_run(bits, 2, g, stream);
}

extern "C" int g4a_gemv_f16(int n_in, int n_out, const float* x, const void* w_f16, float* out, void* stream) {
    const int rc = qgemv_check(16, n_in, n_out, x, (const uint32_t*)w_f16, nullptr, out, 0.0f, 0.0f);
    if (rc != G4A_OK) return rc;
    QgemvArgs g = qgemv_args(n_in, n_out, x, 0.0f, (const uint32_t*)w_f16, nullptr, 0.0f, out);
    return qgemv_run(16, 0, g, stream);
}

extern "C" int g4a_rms_norm(int n_rows, int n, const float* x, float pre, const float* w, const float* res,
                            float mult, float eps, float* out, const float* w2, float q2, int f16_2, float* out2,
                            float* sum2, void* stream) {
    if (n_rows <= 0 || n <= 0 || n_rows > 65535) {
        set_error("n_rows (%d) must be in [1, 65535] and n (%d) positive", n_rows, n);
        return G4A_EINVAL;
    }
    if (!x || !out || (sum2 && !out2) || (w2 && !out2)) {
        set_error("x and out (and out2 when w2 or sum2 is given) must be non-NULL");
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
    a.w2 = w2;
    a.out = out;
    a.out2 = out2;
    a.sum2 = sum2;
    a.n = n;
    a.pre = pre;
    a.mult = mult;
    a.eps = eps;
    a.q2 = q2;
    a.f16_2 = f16_2 != 0;
    if (n > 16384) {
        set_error("n (%d) above 16384", n);
        return G4A_EINVAL;
    }
    const int threads = n > 4096 ? 1024 : 256, per = (n + threads - 1) / threads;
    auto fn = per <= 2 ? rms_kernel<2> : per <= 4 ? rms_kernel<4> : per <= 8 ? rms_kernel<8> : rms_kernel<16>;
    hipLaunchKernelGGL(fn, dim3(n_rows), dim3(threads), 0, (hipStream_t)stream, a);
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

extern "C" int g4a_embed_rows(int bits, int n, const void* table, int64_t n_rows, const int32_t* tok, int n_tok,
                              const float* row_scale, int group, float mult, float* out, void* stream) {
    if (n_tok <= 0 || n_tok > 65535) {
        set_error("n_tok (%d) must be in [1, 65535]", n_tok);
        return G4A_EINVAL;
    }
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
    hipLaunchKernelGGL(embed_kernel, dim3((n + 255) / 256, n_tok), dim3(256), 0, (hipStream_t)stream, bits, n,
                       (const uint32_t*)table, (uint32_t)(n_rows * row_words * 4), row_words, tok, row_scale,
                       (uint32_t)(n_rows * (n / group) * 4), group, mult, out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "embed launch");
    return G4A_OK;
}

extern "C" int g4a_embed(int bits, int n, const void* table, int64_t n_rows, const int32_t* tok,
                         const float* row_scale, int group, float mult, float* out, void* stream) {
    return g4a_embed_rows(bits, n, table, n_rows, tok, 1, row_scale, group, mult, out, stream);
}

extern "C" size_t g4a_softcap_argmax_ws_bytes(int n) {
    return n > 0 ? (size_t)((n + kArgChunk - 1) / kArgChunk) * sizeof(float2) : 0;
}

extern "C" int g4a_softcap_argmax(int n, float* logits, float cap, int32_t* tok, void* ws, size_t ws_bytes,
                                  void* stream) {
    if (n <= 0 || !logits || !tok || !(cap >= 0.0f)) {
        set_error("n must be positive, logits and tok non-NULL, cap >= 0");
        return G4A_EINVAL;
    }
    const int nb = (n + kArgChunk - 1) / kArgChunk;
    if (!ws || ws_bytes < (size_t)nb * sizeof(float2) || (uintptr_t)ws % 8 || (uintptr_t)logits % 16) {
        set_error("softcap_argmax needs %zu workspace bytes (8-byte aligned) and 16-byte aligned logits",
                  (size_t)nb * sizeof(float2));
        return G4A_EWORKSPACE;
    }
    hipLaunchKernelGGL(softcap_part_kernel, dim3(nb), dim3(256), 0, (hipStream_t)stream, n, logits, cap, (float2*)ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "softcap_argmax launch");
    hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, nb, (const float2*)ws, tok);
    e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "argmax launch");
    return G4A_OK;
}
