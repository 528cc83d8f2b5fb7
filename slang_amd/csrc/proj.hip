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
//    tile. srqh_b runs once per layer input (g4a_srqh); the q, k and v GEMMs then share
//    that f16 activation in one grouped launch (g4a_gemm16): K-major ("TN") f16 MFMA tiles
//    fed by a four-stage LDS pipeline, srq_b fused into the q path's store.
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>

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
            h[j] = (half_t)pin(s * ((float)q - zp));  // f16 of the f32 product, as dq_f16 rounds
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
    // norm prologue (PRO): a = srq(rms((pres + rms(pa) * pw1) * pmult) * pw2, pq2) made by
    // every wave from the previous layer's tail; workgroup 0 stores x, a and sum_a
    const float* pa;
    const float* pres;
    const float* pw1;
    const float* pw2;
    float* pxout;
    float* pzout;
    float* psum;
    float pq2, peps, pmult;
};

// NJ chunks of 32 values per lane (hidden <= 2048 * NJ); RPW rows per wave, 4 waves.
// PRO: the input a and its sum come from the norm prologue instead of memory (NJ 1).
// sum over the 256 threads of a workgroup (per wave, then the 4 wave sums in order); every
// thread gets it. Two barriers: red may still be read by the previous call.
__device__ __forceinline__ float wg_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

template <int NJ, int RPW, bool PRO>
__global__ __launch_bounds__(256) void qkv_gemv_kernel(GemvArgs g) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = (blockIdx.x * 4 + wave) * RPW;  // over [q rows | k rows | v rows]
    const int mat = row0 < g.q_dim ? 0 : row0 < g.q_dim + g.kv_dim ? 1 : 2;
    const int r0 = row0 - (mat == 0 ? 0 : mat == 1 ? g.q_dim : g.q_dim + g.kv_dim);
    const int nrows = mat == 0 ? g.q_dim : g.kv_dim;
    const int row_bytes = g.hidden / 2;
    // every operand load first: the prologue's operands, the packed rows, then the input
    // chunks and the sum. Loads return in issue order, so the prologue's operands go out
    // before the rows: its norms and barriers then run while the rows are in flight.
    const rsrc_t ra = make_rsrc(g.a, (uint32_t)g.hidden * 4);
    const rsrc_t rw = make_rsrc(g.bits[mat], (uint32_t)nrows * row_bytes);
    constexpr int PER = 8;  // prologue: thread t holds elements t + 256k of each operand
    float pv[PER], rv[PER], w1v[PER], w2v[PER];
    if constexpr (PRO) {
        const uint32_t nb = (uint32_t)g.hidden * 4;  // past hidden: zeros
        const rsrc_t rpa = make_rsrc(g.pa, nb), rpr = make_rsrc(g.pres, nb), rp1 = make_rsrc(g.pw1, nb),
                     rp2 = make_rsrc(g.pw2, nb);
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int o = 4 * ((int)threadIdx.x + 256 * k);
            pv[k] = bload_f32(rpa, o);
            rv[k] = bload_f32(rpr, o);
            w1v[k] = bload_f32(rp1, o);
            w2v[k] = bload_f32(rp2, o);
        }
    }
    float av[NJ][32];
    u32x4 wv[RPW][NJ];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = lane + 64 * j;  // chunk of the row; past the row end reads zeros
            const int off = c < row_bytes / 16 ? (r0 + r) * row_bytes + 16 * c : 0x7fffffff;
            wv[r][j] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kCpolNT);  // read once: non-temporal
        }
    __builtin_amdgcn_sched_barrier(0);  // no prologue arithmetic (and its waits) above the row loads
    float sa;
    if constexpr (PRO) {
        // once per workgroup: the sums run per thread, then over the workgroup (block_sum); a
        // is staged in LDS, from which lane c of every wave takes elements 32c .. 32c+31. The
        // arithmetic is the rms_kernel's: y = (res + pa / d1 * w1) * mult, z = y / d2 * w2,
        // a = srq(z, q2).
        static_assert(NJ == 1, "the norm prologue covers hidden <= 2048");
        __shared__ float s_a[2048];
        __shared__ float pred[4];
        const int tid = threadIdx.x, n = g.hidden;
        float ss = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; ++k) ss = __builtin_fmaf(pv[k], pv[k], ss);
        const float d1 = sqrtf(wg_sum(ss, pred) / (float)n + g.peps);
        float ss2 = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            rv[k] = (rv[k] + pv[k] / d1 * w1v[k]) * g.pmult;  // x, zeros past hidden
            ss2 = __builtin_fmaf(rv[k], rv[k], ss2);
        }
        const float d2 = sqrtf(wg_sum(ss2, pred) / (float)n + g.peps);
        float s2 = 0.0f;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = tid + 256 * k;
            const float z = srq(rv[k] / d2 * w2v[k], g.pq2);
            if (i < 2048) s_a[i] = i < n ? z : 0.0f;
            s2 += i < n ? z : 0.0f;
            if (blockIdx.x == 0 && i < n) {
                if (g.pxout) g.pxout[i] = rv[k];
                if (g.pzout) g.pzout[i] = z;
            }
        }
        sa = wg_sum(s2, pred);  // its barriers also publish s_a
        if (blockIdx.x == 0 && tid == 0 && g.psum) g.psum[0] = sa;
#pragma unroll
        for (int q4 = 0; q4 < 8; ++q4) {
            const float4v v = *reinterpret_cast<const float4v*>(&s_a[32 * lane + 4 * q4]);
#pragma unroll
            for (int i = 0; i < 4; ++i) av[0][4 * q4 + i] = v[i];
        }
    } else {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int q4 = 0; q4 < 8; ++q4) {
                const float4v v = bload_f32x4(ra, 128 * (lane + 64 * j) + 16 * q4);
#pragma unroll
                for (int i = 0; i < 4; ++i) av[j][4 * q4 + i] = v[i];
            }
        sa = g.sum_a[0];
    }
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

// ---------------------------------------------------------------- f16 GEMM (gemm_tiled)
// srqh_b (kernels_dsl.py:232-242): out = f16(srq(a, s)), 8 values per thread.
__global__ __launch_bounds__(256) void srqh_kernel(const float* __restrict__ a, float s, half_t* __restrict__ out,
                                                   int n8) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const float4v x0 = reinterpret_cast<const float4v*>(a)[2 * i];
    const float4v x1 = reinterpret_cast<const float4v*>(a)[2 * i + 1];
    half8 h;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        h[j] = (half_t)srq(x0[j], s);
        h[4 + j] = (half_t)srq(x1[j], s);
    }
    reinterpret_cast<half8*>(out)[i] = h;
}

// Grouped f16 GEMM: up to three products out_p = A . W_p^T sharing A (the q, k and v
// projections of one layer in one launch). Tiles of 128 tokens x BN outputs, 64-deep k
// stages DMA'd straight from HBM into LDS (buffer_load ... lds, 1 KiB per wave
// instruction), STAGES - 1 stages in flight while the MFMAs run on the oldest. LDS rows are
// 128 B (64 halves, 8 chunks of 16 B); chunk c of row r sits at c ^ ((r >> 1) & 7), so the
// 16 rows of a quarter-wave operand read fall in 16 distinct bank groups. Waves compute
// v_mfma_f32_32x32x16_f16 blocks transposed (D^T = W . A^T) so a lane holds 4 consecutive
// outputs of one token and stores them in one instruction.
//
// Split k: with a workspace, launches with too few tiles to fill the GPU cut k into
// `splits` ranges, one workgroup each. Every workgroup stores its f32 partial tile
// device-coherently, waits for the stores and takes the tile's ticket (a relaxed agent-scope
// atomic); the last of the tile's workgroups to take it adds the partials in split order
// (p0 + p1 + ..., whichever workgroup that is, so the result does not depend on arrival
// order), resets the ticket to zero for the next call and runs the epilogue.
struct Gemm16Args {
    const half_t* a;  // [M][K] f16
    int M, K, mtiles, n_mats;
    const half_t* w[3];  // [N_p][K] f16
    void* out[3];        // [M][N_p] f16, or f32 (srq'd with out_q) when out_f32
    int n[3], out_f32[3];
    float out_q[3], alpha[3];
    int tile_end[3];  // cumulative tiles (n_p / BN) * mtiles
    int tiles, splits;
    unsigned* ticket;  // [tiles], zero between calls
    float* part;       // [tiles][splits][NB * 8][256] float4: the f32 partial tiles
    float gq, uq, oq;  // the gate/up form: geglu_b's steps
    const float* lut;  // ... and the layer's GELU table of the gq grid (gelu_srq), or NULL
};

constexpr int kCpolSC1 = 16;  // device scope: the access bypasses the per-XCD caches
typedef unsigned v4u32 __attribute__((ext_vector_type(4)));

// BN = 64 (outputs per tile) halves the tile for products too narrow to fill the GPU with
// 128 x 128 tiles (N 1536 at M 1024 gives 96 of them for 256 CUs): each wave then covers 32
// outputs x 64 tokens, reading one W block for two MFMAs.
//
// The gate/up form (GEGLU, BN 128): w[0] is the gate matrix, w[1] the up matrix, and a tile
// covers 64 outputs of both: W rows 64 wn + 0..31 are gate rows and 64 wn + 32..63 the up
// rows of the same 32 outputs, so a wave's two 32-output blocks hold gate and up for the same
// (output, token) positions and the epilogue stores geglu_b's code of the two f16 products.
template <int BK, int BN, int STAGES, bool SPLIT, bool GEGLU = false>
__global__ __launch_bounds__(256) void gemm16_kernel(Gemm16Args g) {
    static_assert(!GEGLU || (BN == 128 && !SPLIT), "the gate/up form runs on 128-row tiles");
    static_assert(STAGES >= 2 && STAGES <= 6, "2 to 6 stages");
    constexpr int BM = 128, ROWB = BK * 2;
    constexpr int OPBW = BN * ROWB, OPBA = BM * ROWB;  // operand tile bytes (W, A)
    constexpr int STAGEB = OPBW + OPBA;
    constexpr int CPR = ROWB / 16;          // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;           // rows per 1 KiB wave instruction
    constexpr int WROWS = BN / 4;           // W rows each wave moves per stage
    constexpr int IPOW = WROWS / RPI, IPOA = 32 / RPI;  // instructions per operand and wave per stage
    constexpr int IPS = IPOW + IPOA;        // ... per stage (W and A)
    constexpr int NB = BN / 64;             // 32-output blocks per wave
    // chunk c of row r sits at c ^ swz(r): the rows sharing a 256-byte bank window get
    // distinct chunks, so a quarter-wave operand read touches 16 distinct bank groups
    auto swz = [](int r) { return (r / (256 / ROWB)) % CPR; };
    __shared__ __attribute__((aligned(1024))) char lds[STAGES * STAGEB];  // [stage]{W, A}
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wn = wave & 1, wm = wave >> 1;
    const int l32 = lane & 31, h = lane >> 5;

    // ---- this workgroup's k range, matrix and tile: tiles of one matrix run m-tile-major,
    // so neighbouring workgroups share the rows of A they stream
    const int split = blockIdx.x / g.tiles, tile = blockIdx.x % g.tiles;
    int p = 0, t = tile;
    if (t >= g.tile_end[0]) p = t >= g.tile_end[1] ? 2 : 1;
    if (p > 0) t -= g.tile_end[p - 1];
    constexpr int TN = GEGLU ? BN / 2 : BN;  // outputs a tile covers
    const int ntiles = g.n[p] / TN;
    const int n0 = (t % ntiles) * TN, m0 = (t / ntiles) * BM;
    const int K = g.K, nkall = K / BK;
    const int kt0 = split * nkall / g.splits, nk = (split + 1) * nkall / g.splits - kt0;

    const rsrc_t ra = make_rsrc(g.a, (uint32_t)g.M * K * 2);  // token rows >= M read as zeros
    // the gate/up form: wave w moves gate rows (w even) or up rows (w odd) n0 + 32 (w / 2) ..
    const int wsrc = GEGLU ? (wave & 1) : p;
    const rsrc_t rw = make_rsrc(g.w[wsrc], (uint32_t)g.n[p] * K * 2);
    const int wrow0 = GEGLU ? n0 + 32 * (wave >> 1) - WROWS * wave : n0;  // global row of tile row 0
    // wave w moves W rows WROWS w .. and A rows 32w .. 32w+31, RPI rows (1 KiB) per instruction
    auto issue = [&](int i) {  // stage i of this range = k-step kt0 + i
        char* st = lds + (i % STAGES) * STAGEB;
        const int kb = (kt0 + i) * BK * 2;
#pragma unroll
        for (int j = 0; j < IPOW; ++j) {
            const int r = WROWS * wave + RPI * j + lane / CPR;
            const int c = (lane % CPR) ^ swz(r);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (__attribute__((address_space(3))) void*)(st + (WROWS * wave + RPI * j) * ROWB),
                                                     16, (wrow0 + r) * K * 2 + kb + 16 * c, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < IPOA; ++j) {
            const int r = 32 * wave + RPI * j + lane / CPR;
            const int c = (lane % CPR) ^ swz(r);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (__attribute__((address_space(3))) void*)(st + OPBW + (32 * wave + RPI * j) * ROWB),
                                                     16, (m0 + r) * K * 2 + kb + 16 * c, 0, 0, 0);
        }
    };

    float16v acc[NB][2];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[nb][0] = acc[nb][1] = float16v{};
#pragma unroll
    for (int i = 0; i < STAGES - 1; ++i)
        if (i < nk) issue(i);
    for (int i = 0; i < nk; ++i) {
        // stage i has landed once at most the IPS instructions of each later stage remain
        const int later = min(STAGES - 2, nk - 1 - i);
        static_assert((STAGES - 2) * IPS < 64, "vmcnt holds 6 bits");
        switch (later) {
            case 4: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * IPS) : "memory"); break;
            case 3: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * IPS) : "memory"); break;
            case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * IPS) : "memory"); break;
            case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(IPS) : "memory"); break;
            default: asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        __syncthreads();  // every wave's part of stage i; stage i - 1 fully consumed
        if (i + STAGES - 1 < nk) issue(i + STAGES - 1);
        const char* wl = lds + (i % STAGES) * STAGEB;
        const char* al = wl + OPBW;
        // lane (l32, h) holds k 16s + 8h .. +7 of k-step s; the operands of step s + 1 are
        // read while the MFMAs of step s run (one wave per SIMD hides no LDS latency itself)
        half8 wo[2][NB], ao[2][2];
        auto rd = [&](int s, half8 (&w)[NB], half8 (&x)[2]) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int rw_ = (BN / 2) * wn + 32 * b + l32;
                w[b] = *reinterpret_cast<const half8*>(wl + rw_ * ROWB + 16 * ((2 * s + h) ^ swz(rw_)));
            }
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int ra_ = 64 * wm + 32 * b + l32;
                x[b] = *reinterpret_cast<const half8*>(al + ra_ * ROWB + 16 * ((2 * s + h) ^ swz(ra_)));
            }
        };
        rd(0, wo[0], ao[0]);
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            if (s + 1 < BK / 16) rd(s + 1, wo[(s + 1) & 1], ao[(s + 1) & 1]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) acc[nb][mb] = proj_mfma32(wo[s & 1][nb], ao[s & 1][mb], acc[nb][mb]);
        }
    }

    if constexpr (SPLIT) {
        // publish this split's partial: float4 v of thread tid at [tile][split][v][tid]
        constexpr int NV = NB * 8;
        const size_t tbytes = (size_t)g.splits * NV * 256 * 16;
        const rsrc_t rp = make_rsrc(reinterpret_cast<char*>(g.part) + tile * tbytes, (uint32_t)tbytes);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int v = (nb * 2 + mb) * 4 + q;
                    const float4v x{acc[nb][mb][4 * q], acc[nb][mb][4 * q + 1], acc[nb][mb][4 * q + 2], acc[nb][mb][4 * q + 3]};
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u32, x), rp, ((split * NV + v) * 256 + tid) * 16, 0, kCpolSC1);
                }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this thread's partial stores are done
        __shared__ int s_last;
        __syncthreads();
        if (tid == 0) {
            const unsigned old = __hip_atomic_fetch_add(g.ticket + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = old == (unsigned)g.splits - 1;
            if (last) __hip_atomic_store(g.ticket + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s_last = last;
        }
        __syncthreads();
        if (!s_last) return;
        // the sum in split order, this workgroup's own partial from its registers
        float16v sum[NB][2];
        for (int j = 0; j < g.splits; ++j) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
                    float16v x;
                    if (j == split) {
                        x = acc[nb][mb];
                    } else {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int v = (nb * 2 + mb) * 4 + q;
                            const float4v y = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(
                                                                              rp, ((j * NV + v) * 256 + tid) * 16, 0, kCpolSC1));
#pragma unroll
                            for (int e = 0; e < 4; ++e) x[4 * q + e] = y[e];
                        }
                    }
                    sum[nb][mb] = j == 0 ? x : sum[nb][mb] + x;
                }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[nb][0] = sum[nb][0], acc[nb][1] = sum[nb][1];
    }

    // D^T[n][m]: acc[r] is output n = 8(r/4) + 4h + r%4, token m = l32 of the 32x32 block;
    // the product, times alpha, rounds to f16 (gemm_tiled's f16(alpha * acc)), the q path then
    // applies srq_b
    const int N = g.n[p];
    const bool f32 = g.out_f32[p] != 0;
    const float oq = g.out_q[p], alpha = g.alpha[p];
    // f16 tiles go out through LDS: staged as 128 rows of TN outputs (16 bytes of padding a
    // row, so the 8-byte writes of an instruction fall on distinct banks), then stored as
    // whole row segments, 16 bytes a thread; written straight from the accumulator layout,
    // every store instruction put 16 bytes into each of 32 rows
    constexpr int OS = TN * 2 + 16;
    static_assert(BM * OS <= STAGES * STAGEB, "the staged tile fits the operand stages");
    auto store_staged = [&](half_t* out) {
        __syncthreads();
        constexpr int CH = TN / 8;  // 16-byte chunks a row
#pragma unroll
        for (int i = 0; i < BM * CH / 256; ++i) {
            const int idx = 256 * i + tid, r = idx / CH, ch = idx % CH;
            if (m0 + r < g.M)
                *reinterpret_cast<half8*>(out + (size_t)(m0 + r) * N + n0 + 8 * ch) =
                    *reinterpret_cast<const half8*>(lds + r * OS + 16 * ch);
        }
    };
    if constexpr (GEGLU) {
        __syncthreads();  // every wave is done with the last stage's operands
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const int r = 64 * wm + 32 * mb + l32;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                half4 y;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float gv = (float)(half_t)pin(alpha * acc[0][mb][4 * q + i]);
                    const float uv = (float)(half_t)pin(alpha * acc[1][mb][4 * q + i]);
                    y[i] = geglu_code(gv, uv, g.gq, g.uq, g.oq, g.lut);
                }
                *reinterpret_cast<half4*>(lds + r * OS + (32 * wn + 8 * q + 4 * h) * 2) = y;
            }
        }
        store_staged(reinterpret_cast<half_t*>(g.out[0]));
        return;
    }
    if (!f32) {
        __syncthreads();  // every wave is done with the last stage's operands
#pragma unroll
        for (int mb = 0; mb < 2; ++mb) {
            const int r = 64 * wm + 32 * mb + l32;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    half4 y;
#pragma unroll
                    for (int i = 0; i < 4; ++i) y[i] = (half_t)pin(alpha * acc[nb][mb][4 * q + i]);
                    *reinterpret_cast<half4*>(lds + r * OS + ((BN / 2) * wn + 32 * nb + 8 * q + 4 * h) * 2) = y;
                }
        }
        store_staged(reinterpret_cast<half_t*>(g.out[p]));
        return;
    }
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
        const int m = m0 + 64 * wm + 32 * mb + l32;
        if (m >= g.M) continue;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + (BN / 2) * wn + 32 * nb + 8 * q + 4 * h;
                float4v v;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] = (float)(half_t)pin(alpha * acc[nb][mb][4 * q + i]);
                store4(reinterpret_cast<float*>(g.out[p]) + (size_t)m * N + n, srq4(v, oq));
            }
    }
}

}  // namespace g4a

using namespace g4a;

extern "C" int g4a_srqh(int n, const float* a, float a_in_q, void* out_f16, void* stream) {
    if (n <= 0 || n % 8) {
        set_error("n (%d) must be a positive multiple of 8", n);
        return G4A_EINVAL;
    }
    if (!a || !out_f16 || (((uintptr_t)a | (uintptr_t)out_f16) & 15)) {
        set_error("a and out must be non-NULL and 16-byte aligned");
        return G4A_EINVAL;
    }
    if (!(a_in_q >= 0.0f)) {
        set_error("a_in_q must be >= 0");
        return G4A_EINVAL;
    }
    const int n8 = n / 8;
    hipLaunchKernelGGL(srqh_kernel, dim3((n8 + 255) / 256), dim3(256), 0, (hipStream_t)stream, a, a_in_q,
                       reinterpret_cast<half_t*>(out_f16), n8);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "srqh launch");
    return G4A_OK;
}

// launches whose 128 x 128 tiles number fewer than the CUs run on 128 x 64 tiles: at M 1024
// the N 1536 products (96 wide tiles) went 30.9 -> 26.7 us on them; with 256 or more wide
// tiles (two a CU) the wide ones win (the E2B global layer's q/k/v, 288 wide tiles: 42.3 us
// on 576 narrow ones, 28.2 us on the wide)
constexpr long kGemmNarrowBelow = 256;
// with a workspace, launches of fewer 128 x 64 tiles than CUs (kSplitBelow) split k so that
// about kSplitTarget workgroups run, three a CU (two-stage tiles, 48 KiB of LDS), each over
// at least kSplitMinSteps k-steps. Measured at M 1024 against the unsplit launch: down
// (K 6144, N 1536) 74 -> 42 us, o_proj (K 2048 / 4096) 23.4 -> 19.9 / 50 -> 31 us, the
// per-layer-embedding gate (N 256) 16.2 -> 12.4 us; splitting the 320-tile q/k/v launch
// lost (22 -> 25 us), hence the bound.
constexpr int kSplitBelow = 256, kSplitTarget = 768, kSplitMinSteps = 4, kSplitStages = 2;
// the workspace starts with a ticket word for every tile a split launch can have, so ticket
// words never hold partials of another call
constexpr size_t kTicketBytes = G4A_GEMM_TICKET_BYTES;
static_assert(kSplitBelow * 4 <= kTicketBytes, "a ticket word per split tile");

namespace {
struct GemmPlan {
    int BN, tiles, splits;
    size_t ws_bytes;  // tickets + partials, 0 without a split
};

int gemm_check(int M, int K, const void* a_f16, int n_mats, const g4a_gemm_mat* mats) {
    if (M <= 0 || K <= 0 || K % 64) {
        set_error("M (%d) must be positive and K (%d) a positive multiple of 64", M, K);
        return G4A_EINVAL;
    }
    if (n_mats < 1 || n_mats > 3 || !mats) {
        set_error("n_mats (%d) must be 1, 2 or 3 with a matrix table", n_mats);
        return G4A_EINVAL;
    }
    if (!a_f16 || ((uintptr_t)a_f16 & 15) || (int64_t)(M + 127) * K * 2 > 0x7fffffff) {
        set_error("a must be non-NULL, 16-byte aligned and within 32-bit buffer offsets");
        return G4A_EINVAL;
    }
    for (int i = 0; i < n_mats; ++i) {
        const g4a_gemm_mat* m = &mats[i];
        if (m->n <= 0 || m->n % 128 || !m->w_f16 || !m->out || (((uintptr_t)m->w_f16 | (uintptr_t)m->out) & 15) ||
            (int64_t)m->n * K * 2 > 0x7fffffff || (int64_t)M * m->n > 0x7fffffff || !(m->out_q >= 0.0f)) {
            set_error("matrix %d: n (%d) a positive multiple of 128, w/out non-NULL and 16-byte aligned, "
                      "within 32-bit offsets, out_q >= 0", i, m->n);
            return G4A_EINVAL;
        }
    }
    return G4A_OK;
}

GemmPlan gemm_plan(int M, int K, int n_mats, const g4a_gemm_mat* mats, bool may_split) {
    const int mtiles = (M + 127) / 128;
    long tiles128 = 0;
    for (int i = 0; i < n_mats; ++i) tiles128 += (long)(mats[i].n / 128) * mtiles;
    GemmPlan pl;
    pl.BN = tiles128 < kGemmNarrowBelow ? 64 : 128;  // 64-wide tiles when 128-wide ones leave CUs idle
    pl.tiles = 0;
    for (int i = 0; i < n_mats; ++i) pl.tiles += (mats[i].n / pl.BN) * mtiles;
    pl.splits = 1;
    if (may_split && pl.BN == 64 && pl.tiles < kSplitBelow)
        pl.splits = std::max(1, std::min(K / 64 / kSplitMinSteps, kSplitTarget / pl.tiles));
    pl.ws_bytes = pl.splits > 1 ? kTicketBytes + (size_t)pl.tiles * pl.splits * (pl.BN / 64) * 8 * 256 * 16 : 0;
    return pl;
}

int gemm_run(int M, int K, const void* a_f16, int n_mats, const g4a_gemm_mat* mats, void* ws, size_t ws_bytes,
             void* stream) {
    const int rc = gemm_check(M, K, a_f16, n_mats, mats);
    if (rc != G4A_OK) return rc;
    GemmPlan pl = gemm_plan(M, K, n_mats, mats, ws != nullptr);
    if (pl.splits > 1 && ws_bytes < pl.ws_bytes) {
        set_error("workspace of %zu bytes, this product needs %zu (g4a_gemm16_ws_bytes)", ws_bytes, pl.ws_bytes);
        return G4A_EWORKSPACE;
    }
    if (pl.splits > 1 && ((uintptr_t)ws & 255)) {
        set_error("the workspace must be 256-byte aligned");
        return G4A_EINVAL;
    }
    Gemm16Args g;
    g.a = reinterpret_cast<const half_t*>(a_f16);
    g.M = M;
    g.K = K;
    g.mtiles = (M + 127) / 128;
    g.n_mats = n_mats;
    int tiles = 0;
    for (int i = 0; i < 3; ++i) {
        const g4a_gemm_mat* m = i < n_mats ? &mats[i] : nullptr;
        if (m) tiles += (m->n / pl.BN) * g.mtiles;
        g.w[i] = m ? reinterpret_cast<const half_t*>(m->w_f16) : nullptr;
        g.out[i] = m ? m->out : nullptr;
        g.n[i] = m ? m->n : pl.BN;
        g.out_f32[i] = m ? m->out_f32 : 0;
        g.out_q[i] = m ? m->out_q : 0.0f;
        g.alpha[i] = m && m->alpha != 0.0f ? m->alpha : 1.0f;
        g.tile_end[i] = tiles;
    }
    g.tiles = tiles;
    g.splits = pl.splits;
    g.ticket = pl.splits > 1 ? reinterpret_cast<unsigned*>(ws) : nullptr;
    g.part = pl.splits > 1 ? reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + kTicketBytes) : nullptr;
    const dim3 grid(tiles * pl.splits);
    // LDS 48 / 72 / 64 KiB a workgroup: three / two / two a CU (the 128-wide tiles measured
    // 76 -> 58 us for the decoder's gate/up product with two stages, two a CU, against four
    // stages, one a CU)
    if (pl.splits > 1)
        hipLaunchKernelGGL((gemm16_kernel<64, 64, kSplitStages, true>), grid, dim3(256), 0, (hipStream_t)stream, g);
    else if (pl.BN == 64)
        hipLaunchKernelGGL((gemm16_kernel<64, 64, 3, false>), grid, dim3(256), 0, (hipStream_t)stream, g);
    else
        hipLaunchKernelGGL((gemm16_kernel<64, 128, 2, false>), grid, dim3(256), 0, (hipStream_t)stream, g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "gemm16 launch");
    return G4A_OK;
}
}  // namespace

extern "C" int g4a_gemm16(int M, int K, const void* a_f16, int n_mats, const g4a_gemm_mat* mats, void* stream) {
    return gemm_run(M, K, a_f16, n_mats, mats, nullptr, 0, stream);
}

extern "C" int g4a_gemm16_geglu(int M, int K, const void* a_f16, const void* w_gate_f16, const void* w_up_f16, int n,
                                float gate_q, float up_q, float out_q, void* out_f16, const float* gelu_lut,
                                void* stream) {
    if (M <= 0 || K <= 0 || K % 64 || n <= 0 || n % 64) {
        set_error("M (%d) positive, K (%d) a positive multiple of 64, n (%d) a positive multiple of 64", M, K, n);
        return G4A_EINVAL;
    }
    if (!a_f16 || !w_gate_f16 || !w_up_f16 || !out_f16 ||
        (((uintptr_t)a_f16 | (uintptr_t)w_gate_f16 | (uintptr_t)w_up_f16 | (uintptr_t)out_f16) & 15) ||
        (int64_t)(M + 127) * K * 2 > 0x7fffffff || (int64_t)n * K * 2 > 0x7fffffff || (int64_t)M * n > 0x7fffffff) {
        set_error("a, w_gate, w_up, out non-NULL, 16-byte aligned and within 32-bit offsets");
        return G4A_EINVAL;
    }
    if (!(gate_q >= 0.0f) || !(up_q >= 0.0f) || !(out_q >= 0.0f)) {
        set_error("gate_q, up_q and out_q must be >= 0");
        return G4A_EINVAL;
    }
    Gemm16Args g = {};
    g.a = reinterpret_cast<const half_t*>(a_f16);
    g.M = M;
    g.K = K;
    g.mtiles = (M + 127) / 128;
    g.n_mats = 1;
    g.w[0] = reinterpret_cast<const half_t*>(w_gate_f16);
    g.w[1] = reinterpret_cast<const half_t*>(w_up_f16);
    g.out[0] = out_f16;
    g.n[0] = n;
    g.alpha[0] = 1.0f;
    g.tiles = (n / 64) * g.mtiles;
    g.tile_end[0] = g.tile_end[1] = g.tile_end[2] = g.tiles;
    g.splits = 1;
    g.gq = gate_q;
    g.uq = up_q;
    g.oq = out_q;
    g.lut = gelu_lut;
    hipLaunchKernelGGL((gemm16_kernel<64, 128, 2, false, true>), dim3(g.tiles), dim3(256), 0, (hipStream_t)stream, g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "gemm16_geglu launch");
    return G4A_OK;
}

extern "C" size_t g4a_gemm16_ws_bytes(int M, int K, int n_mats, const g4a_gemm_mat* mats) {
    if (M <= 0 || K <= 0 || K % 64 || n_mats < 1 || n_mats > 3 || !mats) return 0;
    for (int i = 0; i < n_mats; ++i)
        if (mats[i].n <= 0 || mats[i].n % 128) return 0;
    return gemm_plan(M, K, n_mats, mats, true).ws_bytes;
}

extern "C" int g4a_gemm16_ws(int M, int K, const void* a_f16, int n_mats, const g4a_gemm_mat* mats, void* ws,
                             size_t ws_bytes, void* stream) {
    return gemm_run(M, K, a_f16, n_mats, mats, ws, ws_bytes, stream);
}

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

static int qkv_run(int hidden, int q_dim, int kv_dim, const float* a, const float* sum_a,
                   const g4a_norm_in* pro, float* sum_out, const uint32_t* q_bits, const uint32_t* k_bits,
                   const uint32_t* v_bits, const float* scales, float q_out, float k_out, float v_out,
                   float* out_q, float* out_k, float* out_v, void* stream) {
    if (hidden <= 0 || hidden % 32 || hidden > (pro ? 2048 : 4096)) {
        set_error("hidden (%d) must be a positive multiple of 32, at most %d", hidden, pro ? 2048 : 4096);
        return G4A_EINVAL;
    }
    if (pro) {
        if (!pro->a || !pro->res || !pro->w1 || !pro->w2 || pro->f16 || !(pro->q2 >= 0.0f) || !(pro->eps >= 0.0f)) {
            set_error("qkv norm prologue: a, res, w1 and w2 non-NULL, f16 0, q2 and eps >= 0");
            return G4A_EINVAL;
        }
        if (((uintptr_t)pro->a | (uintptr_t)pro->res | (uintptr_t)pro->w1 | (uintptr_t)pro->w2 |
             (uintptr_t)pro->x_out | (uintptr_t)pro->z_out) & 15) {
            set_error("qkv norm prologue: vectors must be 16-byte aligned");
            return G4A_EINVAL;
        }
        // workgroup 0 stores x and z while the others still read a, res and w1
        const size_t vb = (size_t)hidden * sizeof(float);
        for (const void* out : {(const void*)pro->x_out, (const void*)pro->z_out})
            if (overlaps(out, pro->a, vb) || overlaps(out, pro->res, vb) || overlaps(out, pro->w1, vb)) {
                set_error("qkv norm prologue: x_out and z_out must not overlap a, res or w1");
                return G4A_EINVAL;
            }
        a = pro->a;  // checked as the input below; the prologue makes the real one
        sum_a = pro->a;
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
    g.pa = pro ? pro->a : nullptr;
    g.pres = pro ? pro->res : nullptr;
    g.pw1 = pro ? pro->w1 : nullptr;
    g.pw2 = pro ? pro->w2 : nullptr;
    g.pxout = pro ? pro->x_out : nullptr;
    g.pzout = pro ? pro->z_out : nullptr;
    g.psum = sum_out;
    g.pq2 = pro ? pro->q2 : 0.0f;
    g.peps = pro ? pro->eps : 0.0f;
    g.pmult = pro && pro->mult != 0.0f ? pro->mult : 1.0f;
    const int total = q_dim + 2 * kv_dim;  // rows; 2 per wave, 8 per workgroup
    const dim3 grid(total / 8);
    if (pro)
        hipLaunchKernelGGL((qkv_gemv_kernel<1, 2, true>), grid, dim3(256), 0, (hipStream_t)stream, g);
    else if (hidden <= 2048)
        hipLaunchKernelGGL((qkv_gemv_kernel<1, 2, false>), grid, dim3(256), 0, (hipStream_t)stream, g);
    else
        hipLaunchKernelGGL((qkv_gemv_kernel<2, 2, false>), grid, dim3(256), 0, (hipStream_t)stream, g);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "qkv_gemv launch");
    return G4A_OK;
}

extern "C" int g4a_qkv_gemv(int hidden, int q_dim, int kv_dim, const float* a, const float* sum_a,
                            const uint32_t* q_bits, const uint32_t* k_bits, const uint32_t* v_bits,
                            const float* scales, float q_out, float k_out, float v_out, float* out_q,
                            float* out_k, float* out_v, void* stream) {
    return qkv_run(hidden, q_dim, kv_dim, a, sum_a, nullptr, nullptr, q_bits, k_bits, v_bits, scales, q_out, k_out,
                   v_out, out_q, out_k, out_v, stream);
}

extern "C" int g4a_qkv_gemv_norm(int hidden, int q_dim, int kv_dim, const g4a_norm_in* pro, float* sum_out,
                                 const uint32_t* q_bits, const uint32_t* k_bits, const uint32_t* v_bits,
                                 const float* scales, float q_out, float k_out, float v_out, float* out_q,
                                 float* out_k, float* out_v, void* stream) {
    if (!pro) {
        set_error("pro must be non-NULL (g4a_qkv_gemv takes a made input)");
        return G4A_EINVAL;
    }
    return qkv_run(hidden, q_dim, kv_dim, nullptr, nullptr, pro, sum_out, q_bits, k_bits, v_bits, scales, q_out,
                   k_out, v_out, out_q, out_k, out_v, stream);
}
