// Decode attention for gfx950: split-KV flash decoding with an in-kernel
// last-arriver merge.
//
// Reference semantics: attn_101 (gemma4_150/kernels_dsl.py:1537-1749) -- q RMSNorm*gain
// + split-half RoPE (:1593-1615), attended keys [max(0, p+1-W), keyLen) (:1582-1589),
// online softmax per key chunk, partials (acc, m, l) merged by the last chunk to
// finish, which also resets its ticket (:1700-1749); GQA hKv = h / (qH / kvH) (:1581).
//
// MI355X design (not the reference's):
//  * One workgroup per (key split, kv head, sequence) carries ALL G query heads of its
//    GQA group, so each K/V row leaves HBM once. The 4 waves take 16-key blocks in turn.
//  * Scores on the matrix cores: S^T = K . Q^T with v_mfma_f32_16x16x32_f16. A = 16 keys
//    of the block straight from HBM (16 B per lane), B = the G query rows split into an
//    f16 high part (rows 0..G-1) and an f16 low part (rows G..2G-1), so the sum of the
//    two columns is the f32-accurate score; a DPP row shift adds them.
//  * P.V on the VALU from V rows loaded with full 128 B lines (MFMA would need V^T);
//    P reaches the V lanes through a 16xG slice of LDS per wave.
//  * The first block's K/V loads are issued before the q prologue, so the HBM round
//    trip overlaps the norm/RoPE work; rows past the split end are clamped to the last
//    valid row (loaded, then masked), so every load is unconditional.
//  * Waves merge through LDS; splits merge in the last workgroup to finish (one
//    agent-scope release per workgroup, one acquire in the merger), which issues all
//    of its partial loads before it needs them.
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
    uint32_t* tickets;  // [pairs]
    float2* part_ml;    // [pairs][max_splits][G] (m, l)
    float* part_o;      // [pairs][max_splits][G][HD]
    int n_q_heads, n_kv_heads, window, max_splits, chunk;
    float scale_log2, eps, out_q;
};

template <int HD, int G>
struct DecodeShape {
    static constexpr int KSTEPS = HD / 32;        // MFMA k-steps per 16-key tile
    static constexpr int VLANES = HD / 8;         // lanes per V row (8 dims, 16 B each)
    static constexpr int VROWS = 64 / VLANES;     // V rows per load instruction
    static constexpr int VLOADS = 16 / VROWS;     // V load instructions per 16-key block
    static constexpr int LDS_FLOATS = 4 * G * HD; // wave partials
};

__device__ __forceinline__ float4v mfma16(half8 a, half8 b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// K chunk of 8 dims as the f16 MFMA operand; f32 caches are split into high and low
// f16 parts so the score keeps f32 accuracy (the reference's own cache type).
template <typename KVT>
struct KOp;
template <>
struct KOp<half_t> {
    struct raw { half8 h; };
    static __device__ __forceinline__ raw load(const half_t* p) { return raw{*reinterpret_cast<const half8*>(p)}; }
    static __device__ __forceinline__ float4v dot(const raw& k, half8 q, float4v c) { return mfma16(k.h, q, c); }
};
template <>
struct KOp<float> {
    struct raw { float8v f; };
    static __device__ __forceinline__ raw load(const float* p) { return raw{load8(p)}; }
    static __device__ __forceinline__ float4v dot(const raw& k, half8 q, float4v c) {
        const half8 hi = __builtin_convertvector(k.f, half8);
        const half8 lo = __builtin_convertvector(k.f - __builtin_convertvector(hi, float8v), half8);
        return mfma16(lo, q, mfma16(hi, q, c));
    }
};
template <typename KVT>
struct VOp;
template <>
struct VOp<half_t> {
    typedef half8 raw;
    static __device__ __forceinline__ half8 load(const half_t* p) { return *reinterpret_cast<const half8*>(p); }
    static __device__ __forceinline__ float8v cvt(half8 h) { return __builtin_convertvector(h, float8v); }
};
template <>
struct VOp<float> {
    typedef float8v raw;
    static __device__ __forceinline__ float8v load(const float* p) { return load8(p); }
    static __device__ __forceinline__ float8v cvt(float8v f) { return f; }
};

// lane n of each 16-lane row reads lane n+N of the same row
template <int N>
__device__ __forceinline__ float dpp_row_shl(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x100 + N, 0xF, 0xF, false));
}

template <int HD, int G, typename KVT>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
    using Sh = DecodeShape<HD, G>;
    constexpr int KSTEPS = Sh::KSTEPS, VLANES = Sh::VLANES, VROWS = Sh::VROWS, VLOADS = Sh::VLOADS;
    using KO = KOp<KVT>;
    using VO = VOp<KVT>;
    typedef typename KO::raw kraw_t;
    typedef typename VO::raw vraw_t;

    __shared__ __attribute__((aligned(16))) float lds[Sh::LDS_FLOATS];  // wave partials / merge weights
    __shared__ __attribute__((aligned(16))) float lds_p[4][16][G];      // P of the current block, per wave
    __shared__ float lds_m[4][G], lds_l[4][G];
    __shared__ float s_M[G], s_L[G];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int ci = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int pair = b * a.n_kv_heads + kh;

    // ---- attended keys and this workgroup's split (identical in every WG of the pair)
    const int hi = a.key_len[b];
    const int lo = (a.window > 0 && hi > a.window) ? hi - a.window : 0;
    const int active = hi - lo;
    float* outp = a.out + ((size_t)b * a.n_q_heads + (size_t)kh * G) * HD;
    if (active <= 0) {  // no keys: defined output of zeros
        if (ci == 0)
            for (int e = tid; e < G * HD; e += 256) outp[e] = 0.0f;
        return;
    }
    int chunk = a.chunk;  // keys per split (multiple of 16), chosen on the host
    int n_act = (active + chunk - 1) / chunk;
    if (n_act > a.max_splits) {  // a key_len above the host's max_key_len: widen the splits
        chunk = (((active + a.max_splits - 1) / a.max_splits) + 15) & ~15;
        n_act = (active + chunk - 1) / chunk;
    }
    if (ci >= n_act) return;
    const int k0 = lo + ci * chunk;
    const int k1 = min(k0 + chunk, hi);

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

    // ---- q prologue. The G query rows, the gain and this sequence's cos/sin rows are
    // staged through LDS with one coalesced request per thread (all in flight together
    // with the K/V block above). Then rows n < G of the MFMA B operand take the high f16
    // part of head n, rows G..2G-1 the low part, rows >= 2G zero.
    half8 qop[KSTEPS];
    {
        float* sq = lds;                 // [G][HD] q, then [HD] gain, [HD/2] cos, [HD/2] sin
        float* sg = lds + G * HD;
        float* sc_ = sg + HD;
        float* ss_ = sc_ + HD / 2;
        const float4* q4 = reinterpret_cast<const float4*>(a.q + ((size_t)b * a.n_q_heads + (size_t)kh * G) * HD);
        const float4* g4 = reinterpret_cast<const float4*>(a.q_gain ? a.q_gain : kOnes);
        const float4* c4p = reinterpret_cast<const float4*>(a.rcos ? a.rcos + (size_t)b * (HD / 2) : kOnes);
        const float4* s4p = reinterpret_cast<const float4*>(a.rsin ? a.rsin + (size_t)b * (HD / 2) : kZeros);
        constexpr int NQ4 = G * HD / 4, NT4 = NQ4 + HD / 4 + HD / 4;
        float4 st[(NT4 + 255) / 256];
#pragma unroll
        for (int u = 0; u < (NT4 + 255) / 256; ++u) {
            const int idx = tid + 256 * u;
            if (idx < NQ4) st[u] = q4[idx];
            else if (idx < NQ4 + HD / 4) st[u] = g4[idx - NQ4];
            else if (idx < NQ4 + HD / 4 + HD / 8) st[u] = c4p[idx - NQ4 - HD / 4];
            else if (idx < NT4) st[u] = s4p[idx - NQ4 - HD / 4 - HD / 8];
        }
#pragma unroll
        for (int u = 0; u < (NT4 + 255) / 256; ++u)
            if (tid + 256 * u < NT4) reinterpret_cast<float4*>(sq)[tid + 256 * u] = st[u];
        __syncthreads();
        const int h = (n < 2 * G) ? (n % G) : 0;
        float x[KSTEPS][8];
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[s][i] = sq[h * HD + 32 * s + 8 * g + i];
        if (a.q_gain) {
            float ssum = 0.0f;
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
                for (int i = 0; i < 8; ++i) ssum += x[s][i] * x[s][i];
            ssum += xor_shfl(ssum, 16);
            ssum += xor_shfl(ssum, 32);
            const float den = sqrtf(ssum / (float)HD + a.eps);
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
                for (int i = 0; i < 8; ++i) x[s][i] = x[s][i] / den * sg[32 * s + 8 * g + i];
        }
#pragma unroll
        for (int s = 0; s < KSTEPS / 2; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int d = 32 * s + 8 * g + i;
                const float x0 = x[s][i], x1 = x[s + KSTEPS / 2][i];
                x[s][i] = x0 * sc_[d] - x1 * ss_[d];
                x[s + KSTEPS / 2][i] = x1 * sc_[d] + x0 * ss_[d];
            }
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float v = x[s][i] * a.scale_log2;
                const half_t vh = (half_t)v;
                qop[s][i] = n < G ? vh : (n < 2 * G ? (half_t)(v - (float)vh) : (half_t)0.0f);
            }
        __syncthreads();  // the staging area is reused for the wave partials
    }

    // ---- main loop: per wave, 16-key blocks with an online softmax
    float m_run = kNegInf, l_run = 0.0f;  // head n (lanes n < G)
    float acc[G][8];                      // O[h][8 dims of this lane's V column]
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[hh][j] = 0.0f;

    for (; blk < k1; blk += 64) {
        float4v c4 = float4v{0, 0, 0, 0};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) c4 = KO::dot(kr[s], qop[s], c4);
        float sc[4], mloc = kNegInf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float v = c4[i] + dpp_row_shl<G>(c4[i]);  // high + low column
            sc[i] = (blk + 4 * g + i < k1) ? v : kNegInf;
            mloc = fmaxf(mloc, sc[i]);
        }
        mloc = fmaxf(mloc, xor_shfl(mloc, 16));
        mloc = fmaxf(mloc, xor_shfl(mloc, 32));
        const float m_new = fmaxf(m_run, mloc);  // finite: key blk is valid
        const float corr = exp2f(m_run - m_new);
        float ps = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = exp2f(sc[i] - m_new);
            ps += sc[i];
        }
        l_run = l_run * corr + ps;
        m_run = m_new;
        if (n < G) {
#pragma unroll
            for (int i = 0; i < 4; ++i) lds_p[wave][4 * g + i][n] = sc[i];
        }
        float cr[G];
#pragma unroll
        for (int hh = 0; hh < G; ++hh) cr[hh] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, corr), hh));
        vraw_t vcur[VLOADS];
#pragma unroll
        for (int i = 0; i < VLOADS; ++i) vcur[i] = vr[i];
        if (blk + 64 < k1) load_block(blk + 64);  // next block in flight during P.V
#pragma unroll
        for (int hh = 0; hh < G; ++hh)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[hh][j] *= cr[hh];
#pragma unroll
        for (int i = 0; i < VLOADS; ++i) {
            const float8v vf = VO::cvt(vcur[i]);
            const float* pr = &lds_p[wave][VROWS * i + vrow][0];
            float p[G];
#pragma unroll
            for (int hh = 0; hh < G; ++hh) p[hh] = pr[hh];
#pragma unroll
            for (int hh = 0; hh < G; ++hh)
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[hh][j] = fmaf(p[hh], vf[j], acc[hh][j]);
        }
    }

    // ---- wave partial: rows of the same V column summed, then to LDS
    l_run += xor_shfl(l_run, 16);
    l_run += xor_shfl(l_run, 32);
    if constexpr (VROWS == 2) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[hh][j] += xor_shfl(acc[hh][j], 32);
    }
    if (lane < VLANES) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh)
#pragma unroll
            for (int j = 0; j < 8; ++j) lds[(wave * G + hh) * HD + 8 * lane + j] = acc[hh][j];
    }
    if (lane < G) {
        lds_m[wave][lane] = m_run;
        lds_l[wave][lane] = l_run;
    }
    __syncthreads();
    if (tid < G) {
        float M = kNegInf;
        for (int w = 0; w < 4; ++w) M = fmaxf(M, lds_m[w][tid]);
        float L = 0.0f;
        for (int w = 0; w < 4; ++w) L += lds_l[w][tid] * exp2f(lds_m[w][tid] - M);
        s_M[tid] = M;
        s_L[tid] = L;
    }
    __syncthreads();

    const bool single = (n_act == 1);
    float* po = a.part_o + ((size_t)pair * a.max_splits + ci) * (G * HD);
    for (int e = tid; e < G * HD; e += 256) {
        const int hh = e / HD;
        const float M = s_M[hh];
        float o = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) o += lds[w * G * HD + e] * exp2f(lds_m[w][hh] - M);
        if (single)
            outp[e] = srq(o / s_L[hh], a.out_q);
        else
            po[e] = o;
    }
    if (single) return;
    if (tid < G) a.part_ml[((size_t)pair * a.max_splits + ci) * G + tid] = make_float2(s_M[tid], s_L[tid]);

    // ---- publish, take a ticket; the last split of the pair merges all partials.
    // The barrier completes every wave's partial stores; one agent-scope release by
    // thread 0 then makes them visible beyond this XCD's L2, and only the last
    // arriver pays the acquire before reading the other splits' partials.
    __syncthreads();
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const uint32_t t = __hip_atomic_fetch_add(a.tickets + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const int last = (t == (uint32_t)(n_act - 1));
        if (last) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            __hip_atomic_store(a.tickets + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        s_last = last;
    }
    __syncthreads();
    if (!s_last) return;

    // Each thread owns 4 consecutive outputs (float4) and streams the splits 16 at a time.
    // Loads are unconditional (split index clamped; weights of the padding are 0), and the
    // first batch is requested before the weights are computed.
    constexpr int STRIDE4 = G * HD / 4;
    const float4* pob4 = reinterpret_cast<const float4*>(a.part_o + (size_t)pair * a.max_splits * (G * HD));
    const float2* ml = a.part_ml + (size_t)pair * a.max_splits * G;
    float* wts = lds;  // [G][256]; n_act <= max_splits <= 256
    float4 v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) v[u] = pob4[(size_t)min(u, n_act - 1) * STRIDE4 + tid];
    const int n_pad = (n_act + 15) & ~15;
    for (int hh = wave; hh < G; hh += 4) {
        float mloc = kNegInf;
        for (int t = lane; t < n_act; t += 64) mloc = fmaxf(mloc, ml[t * G + hh].x);
        const float M = wave_max(mloc);
        float lsum = 0.0f;
        for (int t = lane; t < n_pad; t += 64) {
            float w = 0.0f;
            if (t < n_act) {
                const float2 w2 = ml[t * G + hh];
                w = exp2f(w2.x - M);
                lsum += w2.y * w;
            }
            wts[hh * 256 + t] = w;
        }
        lsum = wave_sum(lsum);
        if (lane == 0) s_L[hh] = lsum;
    }
    __syncthreads();
    for (int e4 = tid; e4 < STRIDE4; e4 += 256) {
        if (e4 != tid) {
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = pob4[(size_t)min(u, n_act - 1) * STRIDE4 + e4];
        }
        const int hh = (4 * e4) / HD;
        const float* wh = wts + hh * 256;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int t0 = 0;;) {
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const float w = wh[t0 + u];
                o.x = fmaf(w, v[u].x, o.x);
                o.y = fmaf(w, v[u].y, o.y);
                o.z = fmaf(w, v[u].z, o.z);
                o.w = fmaf(w, v[u].w, o.w);
            }
            t0 += 16;
            if (t0 >= n_act) break;
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = pob4[(size_t)min(t0 + u, n_act - 1) * STRIDE4 + e4];
        }
        const float L = s_L[hh];
        float* op = outp + 4 * e4;
        op[0] = srq(o.x / L, a.out_q);
        op[1] = srq(o.y / L, a.out_q);
        op[2] = srq(o.z / L, a.out_q);
        op[3] = srq(o.w / L, a.out_q);
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
    size_t tickets, ml, o, total;
};

static WsLayout ws_layout(const g4a_cfg* cfg, int n_seq, int max_splits) {
    const size_t pairs = (size_t)n_seq * cfg->n_kv_heads;
    const size_t G = cfg->n_q_heads / cfg->n_kv_heads;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    WsLayout L;
    L.tickets = 0;
    L.ml = al(pairs * 4);
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
    a.tickets = (uint32_t*)(w + L.tickets);
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
    return G4A_OK;
}
