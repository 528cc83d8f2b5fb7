// Decode attention for gfx950: split-KV flash decoding; the splits' partials are merged
// by a second kernel.
//
// Reference semantics: attn_101 (gemma4_150/kernels_dsl.py:1537-1749) -- q RMSNorm*gain
// + split-half RoPE (:1593-1615), attended keys [max(0, p+1-W), keyLen) (:1582-1589),
// online softmax per key chunk, partials (acc, m, l) merged by the last chunk to
// finish, which also resets its ticket (:1700-1749); GQA hKv = h / (qH / kvH) (:1581).
//
// MI355X design (not the reference's):
//  * One workgroup per (key split, kv head, sequence) carries ALL G query heads of its
//    GQA group, so each K/V row leaves HBM once. The 4 waves take 16-key blocks in turn.
//  * Both products on the matrix cores, transposed so that no data moves between them:
//    S^T = K . Q^T (v_mfma_f32_16x16x32_f16; A = 16 keys straight from HBM, B = the query
//    rows, f16 high parts in rows 0..G-1 and low parts in rows G..2G-1, so high + low
//    column is the f32-accurate score), then O^T += V^T . P^T (v_mfma_f32_16x16x16_f16).
//    The S^T accumulator layout (lane n,g: keys 4g..4g+3 of column n) is exactly the
//    P^T B-operand layout, and V^T comes from a row-major LDS copy of the block through
//    ds_read_tr16_b64, so P never leaves registers and V is never transposed in memory.
//  * q RMSNorm/RoPE/split is done once per workgroup (one wave per head), its operand
//    loads issued at kernel entry together with the first block's K/V.
//  * Software pipeline without extra registers: once the score MFMAs consumed the K
//    registers and V sits in LDS, the next block's loads reuse both register sets.
//  * Rows past the split end are clamped to the last valid row (loaded, then masked),
//    so every load is unconditional.
//  * Waves merge through LDS. Splits merge in a second, wide kernel (decode_merge_kernel):
//    the kernel boundary publishes the partials, so no workgroup pays a cache-writeback
//    fence or a ticket round trip, and the merge of one (sequence, kv head) is spread over
//    HD/16 workgroups whose threads load all of their splits in one batch. (A last-arriver
//    merge inside this kernel, as attn_101 does, measured 2-4x slower on MI355X: its
//    agent-scope release has to write back the XCD's L2 and the merger then walks every
//    partial serially.)
// Scores are in the log2 domain (q carries scale*log2 e), so the softmax uses exp2.
#include <stdio.h>
#include <stdlib.h>

#include "common.hpp"

namespace g4a {

struct DecodeArgs {
    const int32_t* key_len;
    const float* q;
    const float* q_gain;
    const float* rcos;
    const float* rsin;
    const void* kc;
    const void* vc;
    int64_t seq_stride;
    float* out;
    float2* part_ml;    // [pairs][max_splits][G] (m, l)
    float* part_o;      // [pairs][max_splits][G][HD]
    int n_q_heads, n_kv_heads, window, max_splits, chunk;
    float scale_log2, eps, out_q;
};

template <int HD, int G>
struct DecodeShape {
    static constexpr int KSTEPS = HD / 32;         // score MFMA k-steps per 16-key block
    static constexpr int NDT = HD / 16;            // 16-dim output tiles
    static constexpr int VLANES = HD / 8;          // lanes per V row (8 dims, 16 B each)
    static constexpr int VROWS = 64 / VLANES;      // V rows per load instruction
    static constexpr int VLOADS = 16 / VROWS;      // V load instructions per block
    static constexpr int VSTR = HD + 16;           // LDS V row stride (halves): tr reads conflict-free
    static constexpr int QSTR = HD + 8;            // LDS q row stride (halves)
    static constexpr int V_HALVES = 4 * 16 * VSTR; // per-wave V blocks
    static constexpr int Q_HALVES = 2 * G * QSTR;  // high rows then low rows
    static constexpr int PART_FLOATS = 4 * G * HD; // wave partials / merge weights
    static constexpr int LDS_BYTES_A = V_HALVES * 2 > Q_HALVES * 2 ? V_HALVES * 2 : Q_HALVES * 2;
    static constexpr int LDS_BYTES = LDS_BYTES_A > PART_FLOATS * 4 ? LDS_BYTES_A : PART_FLOATS * 4;
};

__device__ __forceinline__ float4v mfma16x32(half8 a, half8 b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float4v mfma16x16(half4 a, half4 b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// 4 halves of column n of a row-major LDS tile, transposed across each 16-lane group:
// lane n of the group receives element n%4 of the chunks of lanes n/4 + 4j (j < 4).
__device__ __forceinline__ half4 lds_read_tr16(const half_t* p) {
    typedef short short4_ __attribute__((ext_vector_type(4)));
    const short4_ t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_*)(p));
    return __builtin_bit_cast(half4, t);
}

// K chunk of 8 dims as the f16 MFMA operand; f32 caches are split into high and low
// f16 parts so the score keeps f32 accuracy (the reference's own cache type).
template <typename KVT>
struct KOp;
template <>
struct KOp<half_t> {
    struct raw { half8 h; };
    static __device__ __forceinline__ raw load(const half_t* p) { return raw{*reinterpret_cast<const half8*>(p)}; }
    static __device__ __forceinline__ float4v dot(const raw& k, half8 q, float4v c) { return mfma16x32(k.h, q, c); }
};
template <>
struct KOp<float> {
    struct raw { float8v f; };
    static __device__ __forceinline__ raw load(const float* p) { return raw{load8(p)}; }
    static __device__ __forceinline__ float4v dot(const raw& k, half8 q, float4v c) {
        const half8 hi = __builtin_convertvector(k.f, half8);
        const half8 lo = __builtin_convertvector(k.f - __builtin_convertvector(hi, float8v), half8);
        return mfma16x32(lo, q, mfma16x32(hi, q, c));
    }
};
// V chunk of 8 dims, stored to LDS as f16 (f32 caches are rounded, as srqh_b does).
template <typename KVT>
struct VOp;
template <>
struct VOp<half_t> {
    typedef half8 raw;
    static __device__ __forceinline__ half8 load(const half_t* p) { return *reinterpret_cast<const half8*>(p); }
    static __device__ __forceinline__ half8 h(half8 v) { return v; }
};
template <>
struct VOp<float> {
    typedef float8v raw;
    static __device__ __forceinline__ float8v load(const float* p) { return load8(p); }
    static __device__ __forceinline__ half8 h(float8v v) { return __builtin_convertvector(v, half8); }
};

// lane n of each 16-lane row reads lane n+N of the same row
template <int N>
__device__ __forceinline__ float dpp_row_shl(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x100 + N, 0xF, 0xF, false));
}

// Keys attended by sequence b and how they are split: every kernel of a call derives the
// same plan from key_len[b]. Active keys [lo, lo+active); split c covers
// [lo + c*chunk, min(lo + (c+1)*chunk, hi)), c < n_act.
struct SplitPlan {
    int lo, hi, active, chunk, n_act;
};
__device__ __forceinline__ SplitPlan split_plan(const DecodeArgs& a, int b) {
    SplitPlan p;
    p.hi = a.key_len[b];
    p.lo = (a.window > 0 && p.hi > a.window) ? p.hi - a.window : 0;
    p.active = p.hi - p.lo;
    p.chunk = a.chunk;  // keys per split (multiple of 16), chosen on the host
    p.n_act = p.active > 0 ? (p.active + p.chunk - 1) / p.chunk : 0;
    if (p.n_act > a.max_splits) {  // a key_len above the host's max_key_len: widen the splits
        p.chunk = (((p.active + a.max_splits - 1) / a.max_splits) + 15) & ~15;
        p.n_act = (p.active + p.chunk - 1) / p.chunk;
    }
    return p;
}

template <int HD, int G, typename KVT>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
    using Sh = DecodeShape<HD, G>;
    constexpr int KSTEPS = Sh::KSTEPS, NDT = Sh::NDT, VLANES = Sh::VLANES, VROWS = Sh::VROWS;
    constexpr int VLOADS = Sh::VLOADS, VSTR = Sh::VSTR, QSTR = Sh::QSTR;
    using KO = KOp<KVT>;
    using VO = VOp<KVT>;
    typedef typename KO::raw kraw_t;
    typedef typename VO::raw vraw_t;

    // one LDS arena, reused: q rows (prologue) -> V blocks (main loop) -> partials (merges)
    __shared__ __attribute__((aligned(16))) char arena[Sh::LDS_BYTES];
    half_t* sQ = reinterpret_cast<half_t*>(arena);
    half_t* sV = reinterpret_cast<half_t*>(arena);
    float* lds = reinterpret_cast<float*>(arena);
    __shared__ float lds_m[4][G], lds_l[4][G];
    __shared__ float s_M[G], s_L[G], s_W[4][G];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int ci = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int pair = b * a.n_kv_heads + kh;

    // ---- q operand loads first: they depend on nothing but the sequence and kv head
    constexpr int QP = HD / 128;  // elements per lane in each half of a head row
    const int d0 = QP * lane;     // this lane: dims d0.. and d0+HD/2..
    float qx[2][QP], qgv[2][QP], qcv[QP], qsv[QP];
    {
        const float* qb = a.q + ((size_t)b * a.n_q_heads + (size_t)kh * G) * HD;
        const float* gp = a.q_gain ? a.q_gain : kOnes;
        const float* cp = a.rcos ? a.rcos + (size_t)b * (HD / 2) : kOnes;
        const float* sp = a.rsin ? a.rsin + (size_t)b * (HD / 2) : kZeros;
        const int hh = wave < G ? wave : 0;
#pragma unroll
        for (int e = 0; e < QP; ++e) {
            qx[0][e] = qb[hh * HD + d0 + e];
            qx[1][e] = qb[hh * HD + HD / 2 + d0 + e];
            qgv[0][e] = gp[d0 + e];
            qgv[1][e] = gp[HD / 2 + d0 + e];
            qcv[e] = cp[d0 + e];
            qsv[e] = sp[d0 + e];
        }
    }

    // ---- attended keys and this workgroup's split
    const SplitPlan sp = split_plan(a, b);
    float* outp = a.out + ((size_t)b * a.n_q_heads + (size_t)kh * G) * HD;
    if (sp.active <= 0) {  // no keys: defined output of zeros
        if (ci == 0)
            for (int e = tid; e < G * HD; e += 256) outp[e] = 0.0f;
        return;
    }
    const int n_act = sp.n_act;
    if (ci >= n_act) return;
    const int k0 = sp.lo + ci * sp.chunk;
    const int k1 = min(k0 + sp.chunk, sp.hi);

    // ---- block loads: K in the MFMA A layout (lane n,g: key n, dims 32s+8g..), V rows
    const size_t rstride = (size_t)a.n_kv_heads * HD;
    const KVT* kbase = reinterpret_cast<const KVT*>(a.kc) + (size_t)b * a.seq_stride + (size_t)kh * HD + 8 * g;
    const KVT* vbase = reinterpret_cast<const KVT*>(a.vc) + (size_t)b * a.seq_stride + (size_t)kh * HD +
                       8 * (lane % VLANES);
    const int vrow = lane / VLANES;
    kraw_t kr[KSTEPS];
    vraw_t vr[VLOADS];
    auto load_block = [&](int blk) {
        const int kk = min(blk + n, k1 - 1);
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) kr[s] = KO::load(kbase + (size_t)kk * rstride + 32 * s);
#pragma unroll
        for (int i = 0; i < VLOADS; ++i) {
            const int kv = min(blk + VROWS * i + vrow, k1 - 1);
            vr[i] = VO::load(vbase + (size_t)kv * rstride);
        }
    };
    int blk = k0 + wave * 16;
    if (blk < k1) load_block(blk);  // in flight during the q prologue

    // ---- q prologue: wave w prepares head w (and w+4): RMSNorm*gain, RoPE, scale*log2 e,
    // split into f16 high/low rows of the B operand, staged in LDS.
#pragma unroll
    for (int hh = wave; hh < G; hh += 4) {
        float x[2][QP];
        if (hh != wave) {  // G = 8: second head of this wave
            const float* qb = a.q + ((size_t)b * a.n_q_heads + (size_t)kh * G + hh) * HD;
#pragma unroll
            for (int e = 0; e < QP; ++e) {
                qx[0][e] = qb[d0 + e];
                qx[1][e] = qb[HD / 2 + d0 + e];
            }
        }
#pragma unroll
        for (int e = 0; e < QP; ++e) {
            x[0][e] = qx[0][e];
            x[1][e] = qx[1][e];
        }
        if (a.q_gain) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < QP; ++e) ss += x[0][e] * x[0][e] + x[1][e] * x[1][e];
            const float rs = 1.0f / sqrtf(wave_sum(ss) / (float)HD + a.eps);  // attn_101's q * nscale * w
#pragma unroll
            for (int e = 0; e < QP; ++e) {
                x[0][e] = x[0][e] * rs * qgv[0][e];
                x[1][e] = x[1][e] * rs * qgv[1][e];
            }
        }
#pragma unroll
        for (int e = 0; e < QP; ++e) {
            const float x0 = x[0][e], x1 = x[1][e];
            const float r0 = (x0 * qcv[e] - x1 * qsv[e]) * a.scale_log2;
            const float r1 = (x1 * qcv[e] + x0 * qsv[e]) * a.scale_log2;
            const half_t h0 = (half_t)r0, h1 = (half_t)r1;
            sQ[hh * QSTR + d0 + e] = h0;
            sQ[hh * QSTR + HD / 2 + d0 + e] = h1;
            sQ[(G + hh) * QSTR + d0 + e] = (half_t)(r0 - (float)h0);
            sQ[(G + hh) * QSTR + HD / 2 + d0 + e] = (half_t)(r1 - (float)h1);
        }
    }
    __syncthreads();
    half8 qop[KSTEPS];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s)
        qop[s] = n < 2 * G ? *reinterpret_cast<const half8*>(&sQ[n * QSTR + 32 * s + 8 * g])
                           : half8{0, 0, 0, 0, 0, 0, 0, 0};
    __syncthreads();  // the arena now holds the V blocks

    // ---- main loop: per wave, 16-key blocks with an online softmax per head column
    half_t* myV = sV + wave * 16 * VSTR;
    float m_run = kNegInf, l_run = 0.0f;  // column n (heads: n < G)
    float4v oacc[NDT];                    // O^T[16dt + 4g + i][column n]
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = float4v{0, 0, 0, 0};

    for (; blk < k1; blk += 64) {
#pragma unroll
        for (int i = 0; i < VLOADS; ++i)
            *reinterpret_cast<half8*>(&myV[(VROWS * i + vrow) * VSTR + 8 * (lane % VLANES)]) = VO::h(vr[i]);
        float4v c4 = float4v{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) c4 = KO::dot(kr[s], qop[s], c4);
        if (blk + 64 < k1) load_block(blk + 64);  // next block in flight during softmax and P.V
        float sc[4], mloc = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = c4[i] + dpp_row_shl<G>(c4[i]);  // high + low column
            sc[i] = (n < G && blk + 4 * g + i < k1) ? v : kNegInf;
            mloc = fmaxf(mloc, sc[i]);
        }
        mloc = max32(max16(mloc));
        const float m_new = fmaxf(m_run, mloc);            // finite for heads: key blk is valid
        const float m_use = (m_new == kNegInf) ? 0.0f : m_new;  // padding columns stay at zero
        half4 pb;
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float p = fexp2(sc[i] - m_use);
            ps += p;
            pb[i] = (half_t)p;
        }
        const float corr = fexp2(m_run - m_use);
        l_run = l_run * corr + ps;
        m_run = m_new;
        if (__any(corr != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= corr;
        }
        // O^T += V^T . P^T : lane n of group g supplies V[key 4g + n/4][16dt + 4(n%4) ..]
        const half_t* vrd = myV + (4 * g + (n >> 2)) * VSTR + 4 * (n & 3);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma16x16(lds_read_tr16(vrd + 16 * dt), pb, oacc[dt]);
    }

    // ---- wave partial: column sums, then the head columns to LDS
    l_run = add32(add16(l_run));
    __syncthreads();  // every wave is done with its V block: the arena takes the partials
    if (n < G) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) lds[(wave * G + n) * HD + 16 * dt + 4 * g + i] = oacc[dt][i];
        if (g == 0) {
            lds_m[wave][n] = m_run;
            lds_l[wave][n] = l_run;
        }
    }
    __syncthreads();
    if (tid < G) {
        float M = kNegInf;
        for (int w = 0; w < 4; ++w) M = fmaxf(M, lds_m[w][tid]);
        float L = 0.0f;
        for (int w = 0; w < 4; ++w) {
            const float wt = fexp2(lds_m[w][tid] - M);
            s_W[w][tid] = wt;
            L += lds_l[w][tid] * wt;
        }
        s_M[tid] = M;
        s_L[tid] = L;
    }
    __syncthreads();

    const bool single = (n_act == 1);
    float* po = a.part_o + ((size_t)pair * a.max_splits + ci) * (G * HD);
    for (int e = tid; e < G * HD; e += 256) {
        const int hh = e / HD;
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) o += lds[w * G * HD + e] * s_W[w][hh];
        if (single)
            outp[e] = srq(o * (1.0f / s_L[hh]), a.out_q);
        else
            po[e] = o;
    }
    if (single) return;
    if (tid < G) a.part_ml[((size_t)pair * a.max_splits + ci) * G + tid] = make_float2(s_M[tid], s_L[tid]);
}

// Merge of the split partials: out = sum_c o_c 2^(m_c - M) / sum_c l_c 2^(m_c - M), M = max_c m_c
// (the flash-decoding identity attn_101 applies in its last chunk, kernels_dsl.py:1717-1749).
// One workgroup per (64 output dims, kv head, sequence): thread (split group sg, dim d) loads
// splits c = sg, sg+4, ... of its output element in one batch of up to 16 (loads are
// unconditional: the index is clamped and padded splits weigh 0), then the four split groups
// are summed through LDS. Sequences whose keys fit one split were finished by decode_kernel.
template <int HD, int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    constexpr int E = G * HD;
    __shared__ float wts[256];
    __shared__ float red[4][64];
    __shared__ float s_red[4], s_L;
    const int tid = threadIdx.x, lane = tid & 63, sg = tid >> 6;
    const int e = blockIdx.x * 64 + lane, hh = (blockIdx.x * 64) / HD;
    const int kh = blockIdx.y, b = blockIdx.z, pair = b * a.n_kv_heads + kh;
    const SplitPlan sp = split_plan(a, b);
    const int n_act = sp.n_act;
    if (n_act <= 1) return;
    const float* po = a.part_o + (size_t)pair * a.max_splits * E + e;
    const float2* ml = a.part_ml + (size_t)pair * a.max_splits * G + hh;
    float v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = po[(size_t)min(sg + 4 * u, n_act - 1) * E];
    // weights of every split for this head
    const float2 mlt = ml[(size_t)min(tid, n_act - 1) * G];
    float mloc = tid < n_act ? mlt.x : kNegInf;
    mloc = wave_max(mloc);
    if (lane == 0) s_red[sg] = mloc;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float w = tid < n_act ? fexp2(mlt.x - M) : 0.0f;
    wts[tid] = w;
    const float lw = wave_sum(w * (tid < n_act ? mlt.y : 0.0f));
    __syncthreads();
    if (lane == 0) s_red[sg] = lw;
    __syncthreads();
    if (tid == 0) s_L = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    float o = 0.0f;
#pragma unroll
    for (int u = 0; u < 16; ++u) o = fmaf(wts[min(sg + 4 * u, 255)] * (sg + 4 * u < n_act ? 1.0f : 0.0f), v[u], o);
    for (int c0 = 64; c0 < n_act; c0 += 64) {  // more than 64 splits: further batches
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = po[(size_t)min(c0 + sg + 4 * u, n_act - 1) * E];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int c = c0 + sg + 4 * u;
            o = fmaf(c < n_act ? wts[c] : 0.0f, v[u], o);
        }
    }
    red[sg][lane] = o;
    __syncthreads();
    if (sg == 0) {
        const float t = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
        a.out[((size_t)b * a.n_q_heads + (size_t)kh * G) * HD + e] = srq(t * (1.0f / s_L), a.out_q);
    }
}

// ---------------------------------------------------------------- host side
static int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v && *v ? atoi(v) : dflt;
}

// Keys per split: spread the worst-case work (every sequence at max_key_len) over about
// G4A_DECODE_TARGET_WGS workgroups, but never below G4A_DECODE_MIN_CHUNK keys, so the
// partial (G*hd floats) stays small next to the K/V it summarises.
static int decode_chunk(const g4a_cfg* cfg, int n_seq, int max_key_len) {
    const long pairs = (long)n_seq * cfg->n_kv_heads;
    long max_active = max_key_len;
    if (cfg->window > 0 && (long)cfg->window < max_active) max_active = cfg->window;
    const long target = env_int("G4A_DECODE_TARGET_WGS", 1024);
    long min_chunk = env_int("G4A_DECODE_MIN_CHUNK", 32);
    long chunk = (max_active * pairs + target - 1) / target;
    if (chunk < min_chunk) chunk = min_chunk;
    if ((max_active + chunk - 1) / chunk > 256) chunk = (max_active + 255) / 256;
    return (int)((chunk + 15) & ~15L);
}

static int decode_splits(const g4a_cfg* cfg, int n_seq, int max_key_len) {
    long max_active = max_key_len;
    if (cfg->window > 0 && (long)cfg->window < max_active) max_active = cfg->window;
    const int chunk = decode_chunk(cfg, n_seq, max_key_len);
    const long s = (max_active + chunk - 1) / chunk;
    return (int)(s < 1 ? 1 : s);
}

struct WsLayout {
    size_t ml, o, total;
};

static WsLayout ws_layout(const g4a_cfg* cfg, int n_seq, int max_splits) {
    const size_t pairs = (size_t)n_seq * cfg->n_kv_heads;
    const size_t G = cfg->n_q_heads / cfg->n_kv_heads;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    WsLayout L;
    L.ml = 0;
    L.o = L.ml + al(pairs * max_splits * G * sizeof(float2));
    L.total = L.o + pairs * max_splits * G * cfg->head_dim * sizeof(float);
    return L;
}

typedef void (*decode_fn)(DecodeArgs);

template <int HD, int G>
static decode_fn pick_kv(bool f32) {
    return f32 ? decode_kernel<HD, G, float> : decode_kernel<HD, G, half_t>;
}
template <int HD>
static decode_fn pick_g(int G, bool f32) {
    switch (G) {
        case 1: return pick_kv<HD, 1>(f32);
        case 2: return pick_kv<HD, 2>(f32);
        case 4: return pick_kv<HD, 4>(f32);
        case 8: return pick_kv<HD, 8>(f32);
    }
    return nullptr;
}
template <int HD>
static decode_fn pick_merge(int G) {
    switch (G) {
        case 1: return decode_merge_kernel<HD, 1>;
        case 2: return decode_merge_kernel<HD, 2>;
        case 4: return decode_merge_kernel<HD, 4>;
        case 8: return decode_merge_kernel<HD, 8>;
    }
    return nullptr;
}

}  // namespace g4a

using namespace g4a;

extern "C" size_t g4a_decode_ws_bytes(const g4a_cfg* cfg, int n_seq, int max_key_len) {
    if (!check_cfg(cfg, true) || n_seq <= 0 || max_key_len <= 0) return 0;
    return ws_layout(cfg, n_seq, decode_splits(cfg, n_seq, max_key_len)).total;
}

extern "C" int g4a_decode(const g4a_cfg* cfg, int n_seq, int max_key_len, const int32_t* key_len,
                          const float* q, const float* q_gain, const float* rope_cos,
                          const float* rope_sin, const void* k_cache, const void* v_cache,
                          int64_t seq_stride, float* out, void* ws, size_t ws_bytes, void* stream) {
    if (!check_cfg(cfg, true)) return G4A_EINVAL;
    if (n_seq <= 0 || max_key_len <= 0) {
        set_error("n_seq (%d) and max_key_len (%d) must be positive", n_seq, max_key_len);
        return G4A_EINVAL;
    }
    if (!key_len || !q || !k_cache || !v_cache || !out) {
        set_error("key_len, q, k_cache, v_cache and out must be non-NULL");
        return G4A_EINVAL;
    }
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) {
        set_error("rope_cos and rope_sin must both be given or both be NULL");
        return G4A_EINVAL;
    }
    const int HD = (int)cfg->head_dim, G = (int)(cfg->n_q_heads / cfg->n_kv_heads);
    if (HD != 256 && HD != 512) {
        set_error("head_dim %d not supported (256 or 512)", HD);
        return G4A_EUNSUPPORTED;
    }
    const bool f32 = (cfg->flags & G4A_KV_F32) != 0;
    const size_t esz = f32 ? 4 : 2;
    if (((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)q | (uintptr_t)out) % 16 ||
        (q_gain && (uintptr_t)q_gain % 16) || (rope_cos && ((uintptr_t)rope_cos | (uintptr_t)rope_sin) % 16) ||
        (seq_stride * esz) % 16) {
        set_error("q, q_gain, rope tables, caches, out and seq_stride*elem_size must be 16-byte aligned");
        return G4A_EINVAL;
    }
    if (n_seq > 1 && seq_stride < (int64_t)cfg->n_kv_heads * HD) {
        set_error("seq_stride %lld smaller than one cache row", (long long)seq_stride);
        return G4A_EINVAL;
    }
    const int splits = decode_splits(cfg, n_seq, max_key_len);
    const WsLayout L = ws_layout(cfg, n_seq, splits);
    if (!ws || ws_bytes < L.total || ((uintptr_t)ws % 256)) {
        set_error("decode workspace needs %zu bytes (256-byte aligned), got %zu", L.total, ws_bytes);
        return G4A_EWORKSPACE;
    }
    if ((int64_t)n_seq * cfg->n_kv_heads > 65535) {
        set_error("n_seq*n_kv_heads too large");
        return G4A_EINVAL;
    }
    DecodeArgs a;
    a.key_len = key_len;
    a.q = q;
    a.q_gain = q_gain;
    a.rcos = rope_cos;
    a.rsin = rope_sin;
    a.kc = k_cache;
    a.vc = v_cache;
    a.seq_stride = seq_stride;
    a.out = out;
    char* w = (char*)ws;
    a.part_ml = (float2*)(w + L.ml);
    a.part_o = (float*)(w + L.o);
    a.n_q_heads = (int)cfg->n_q_heads;
    a.n_kv_heads = (int)cfg->n_kv_heads;
    a.window = (int)cfg->window;
    a.max_splits = splits;
    a.chunk = decode_chunk(cfg, n_seq, max_key_len);
    a.scale_log2 = cfg->scale * kLog2e;
    a.eps = cfg->eps;
    a.out_q = cfg->out_q;
    decode_fn fn = HD == 256 ? pick_g<256>(G, f32) : pick_g<512>(G, f32);
    if (!fn) {
        set_error("no decode kernel for group size %d", G);
        return G4A_EUNSUPPORTED;
    }
    dim3 grid(splits, cfg->n_kv_heads, n_seq);
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, (hipStream_t)stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "decode launch");
    if (splits > 1) {
        decode_fn mf = HD == 256 ? pick_merge<256>(G) : pick_merge<512>(G);
        hipLaunchKernelGGL(mf, dim3(G * HD / 64, cfg->n_kv_heads, n_seq), dim3(256), 0, (hipStream_t)stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return hip_error(e, "decode merge launch");
    }
    return G4A_OK;
}
