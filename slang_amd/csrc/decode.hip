// Decode attention for gfx950: split-KV flash decoding with an in-kernel
// last-arriver merge.
//
// Reference semantics: attn_101 (gemma4_150/kernels_dsl.py:1537-1749) -- q RMSNorm*gain
// + split-half RoPE (:1593-1615), attended keys [max(0, p+1-W), keyLen) (:1582-1589),
// online softmax per key chunk, partials (acc, m, l) merged by the last chunk to
// finish, which also resets its ticket (:1700-1749); GQA hKv = h / (qH / kvH) (:1581).
//
// MI355X design (not the reference's): one workgroup per (key split, kv head, sequence)
// carries ALL query heads of its GQA group, so each K/V row is read from HBM once.
// Within a workgroup the 4 waves take 16-key blocks round-robin; each wave keeps its
// own online softmax in registers and the waves are merged through LDS. Each K/V row
// (hd f16 = 512 B at hd 256) is read by LPK lanes with 16 B loads, so every load
// instruction moves full 128 B lines; the per-key dot products are reduced with DPP
// row rotations. Scores live in the log2 domain (q is pre-scaled by scale*log2 e)
// so the softmax uses exp2.
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
    static constexpr int LPK0 = G * HD / 64;                  // lanes per key so that q+acc fit
    static constexpr int LPK = LPK0 < 16 ? 16 : (LPK0 > 64 ? 64 : LPK0);
    static constexpr int KPS = 64 / LPK;                      // keys per wave step
    static constexpr int NCH = HD / (8 * LPK);                // 8-element chunks per lane
    static constexpr int NE = 8 * NCH;                        // elements per lane
    static constexpr int NS0 = 16 / KPS;
    static constexpr int NS = (NS0 * G > 32) ? (32 / G) : NS0;  // wave steps per block
    static constexpr int BK = KPS * NS;                       // keys per wave block
    static constexpr int LDS_FLOATS = 4 * G * HD;             // wave partials (aliases q)
};

template <int LPK>
__device__ __forceinline__ float key_sum(float x) {
    x = row16_sum(x);
    if constexpr (LPK >= 32) x += xor_shfl(x, 16);
    if constexpr (LPK >= 64) x += xor_shfl(x, 32);
    return x;
}

// reduce across the 64/LPK rows of a wave (lanes holding different keys)
template <int LPK>
__device__ __forceinline__ float rows_max(float x) {
    if constexpr (LPK <= 16) x = fmaxf(x, xor_shfl(x, 16));
    if constexpr (LPK <= 32) x = fmaxf(x, xor_shfl(x, 32));
    return x;
}
template <int LPK>
__device__ __forceinline__ float rows_sum(float x) {
    if constexpr (LPK <= 16) x += xor_shfl(x, 16);
    if constexpr (LPK <= 32) x += xor_shfl(x, 32);
    return x;
}

template <typename KVT>
struct RawChunk;
template <>
struct RawChunk<half_t> {
    typedef half8 type;
    static __device__ __forceinline__ half8 load(const half_t* p) { return *reinterpret_cast<const half8*>(p); }
    static __device__ __forceinline__ half8 zero() { return half8{0, 0, 0, 0, 0, 0, 0, 0}; }
    static __device__ __forceinline__ float8v cvt(half8 h) { return __builtin_convertvector(h, float8v); }
};
template <>
struct RawChunk<float> {
    typedef float8v type;
    static __device__ __forceinline__ float8v load(const float* p) { return load8(p); }
    static __device__ __forceinline__ float8v zero() { return float8v{0, 0, 0, 0, 0, 0, 0, 0}; }
    static __device__ __forceinline__ float8v cvt(float8v f) { return f; }
};

template <int HD, int G, typename KVT>
__global__ __launch_bounds__(256) void decode_kernel(DecodeArgs a) {
    using Sh = DecodeShape<HD, G>;
    constexpr int LPK = Sh::LPK, KPS = Sh::KPS, NCH = Sh::NCH, NE = Sh::NE, NS = Sh::NS, BK = Sh::BK;
    using RC = RawChunk<KVT>;
    typedef typename RC::type raw_t;

    __shared__ __attribute__((aligned(16))) float lds[Sh::LDS_FLOATS];  // [4][G][HD] wave partials; q at start
    __shared__ float lds_m[4][G], lds_l[4][G];
    __shared__ float s_M[G], s_L[G];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane / LPK, c = lane % LPK;
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

    // ---- q prologue: RMSNorm*gain, RoPE, scale*log2e, into LDS [G][HD]
    {
        const float* qb = a.q + ((size_t)b * a.n_q_heads + (size_t)kh * G) * HD;
        constexpr int PER = HD / 64;
        for (int hh = wave; hh < G; hh += 4) {
            float x[PER];
#pragma unroll
            for (int m = 0; m < PER; ++m) x[m] = qb[hh * HD + lane + 64 * m];
            if (a.q_gain) {
                float ss = 0.0f;
#pragma unroll
                for (int m = 0; m < PER; ++m) ss += x[m] * x[m];
                ss = wave_sum(ss);
                const float den = sqrtf(ss / (float)HD + a.eps);
#pragma unroll
                for (int m = 0; m < PER; ++m) x[m] = x[m] / den * a.q_gain[lane + 64 * m];
            }
            if (a.rcos) {
                const float* cs = a.rcos + (size_t)b * (HD / 2);
                const float* sn = a.rsin + (size_t)b * (HD / 2);
#pragma unroll
                for (int m = 0; m < PER / 2; ++m) {
                    const int d = lane + 64 * m;
                    const float x0 = x[m], x1 = x[m + PER / 2];
                    x[m] = x0 * cs[d] - x1 * sn[d];
                    x[m + PER / 2] = x1 * cs[d] + x0 * sn[d];
                }
            }
#pragma unroll
            for (int m = 0; m < PER; ++m) lds[hh * HD + lane + 64 * m] = x[m] * a.scale_log2;
        }
    }
    __syncthreads();
    float qv[G][NE];
#pragma unroll
    for (int hh = 0; hh < G; ++hh)
#pragma unroll
        for (int j = 0; j < NCH; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) qv[hh][8 * j + i] = lds[hh * HD + 8 * LPK * j + 8 * c + i];
    __syncthreads();  // the q region is reused for the wave partials below

    // ---- main loop: 16-key-ish blocks per wave, online softmax in registers
    const int rstride = a.n_kv_heads * HD;
    const KVT* kbase = reinterpret_cast<const KVT*>(a.kc) + (size_t)b * a.seq_stride + (size_t)kh * HD + 8 * c;
    const KVT* vbase = reinterpret_cast<const KVT*>(a.vc) + (size_t)b * a.seq_stride + (size_t)kh * HD + 8 * c;

    float m_run[G], l_run[G], acc[G][NE];
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        m_run[hh] = kNegInf;
        l_run[hh] = 0.0f;
#pragma unroll
        for (int e = 0; e < NE; ++e) acc[hh][e] = 0.0f;
    }

    // K/V of the next block are loaded while the current one is processed
    raw_t kr[NS][NCH], vr[NS][NCH];
    auto load_block = [&](int blk, raw_t (&kk)[NS][NCH], raw_t (&vv)[NS][NCH]) {
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            const int key = blk + t * KPS + r;
            const bool ok = key < k1;
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                const size_t off = (size_t)key * rstride + 8 * LPK * j;
                kk[t][j] = ok ? RC::load(kbase + off) : RC::zero();
                vv[t][j] = ok ? RC::load(vbase + off) : RC::zero();
            }
        }
    };
    int blk = k0 + wave * BK;
    if (blk < k1) load_block(blk, kr, vr);
    for (; blk < k1; blk += 4 * BK) {
        raw_t kn[NS][NCH], vn[NS][NCH];
        load_block(blk + 4 * BK, kn, vn);  // keys >= k1 load nothing
        float s[NS][G];
#pragma unroll
        for (int t = 0; t < NS; ++t) {
            float part[G];
#pragma unroll
            for (int hh = 0; hh < G; ++hh) part[hh] = 0.0f;
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                const float8v kf = RC::cvt(kr[t][j]);
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int hh = 0; hh < G; ++hh) part[hh] = fmaf(qv[hh][8 * j + i], kf[i], part[hh]);
            }
            const bool ok = blk + t * KPS + r < k1;
#pragma unroll
            for (int hh = 0; hh < G; ++hh) {
                const float v = key_sum<LPK>(part[hh]);
                s[t][hh] = ok ? v : kNegInf;
            }
        }
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            float mb = s[0][hh];
#pragma unroll
            for (int t = 1; t < NS; ++t) mb = fmaxf(mb, s[t][hh]);
            mb = rows_max<LPK>(mb);
            const float m_new = fmaxf(m_run[hh], mb);  // finite: key blk is always valid
            const float corr = exp2f(m_run[hh] - m_new);
            float ps = 0.0f;
#pragma unroll
            for (int t = 0; t < NS; ++t) {
                s[t][hh] = exp2f(s[t][hh] - m_new);
                ps += s[t][hh];
            }
            l_run[hh] = l_run[hh] * corr + ps;
            m_run[hh] = m_new;
#pragma unroll
            for (int e = 0; e < NE; ++e) acc[hh][e] *= corr;
        }
#pragma unroll
        for (int t = 0; t < NS; ++t)
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                const float8v vf = RC::cvt(vr[t][j]);
#pragma unroll
                for (int i = 0; i < 8; ++i)
#pragma unroll
                    for (int hh = 0; hh < G; ++hh) acc[hh][8 * j + i] = fmaf(s[t][hh], vf[i], acc[hh][8 * j + i]);
            }
#pragma unroll
        for (int t = 0; t < NS; ++t)
#pragma unroll
            for (int j = 0; j < NCH; ++j) {
                kr[t][j] = kn[t][j];
                vr[t][j] = vn[t][j];
            }
    }

    // ---- wave partial: sum over rows (lanes with different keys), then to LDS
#pragma unroll
    for (int hh = 0; hh < G; ++hh) {
        l_run[hh] = rows_sum<LPK>(l_run[hh]);
#pragma unroll
        for (int e = 0; e < NE; ++e) acc[hh][e] = rows_sum<LPK>(acc[hh][e]);
    }
    if (r == 0) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh)
#pragma unroll
            for (int j = 0; j < NCH; ++j)
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    lds[(wave * G + hh) * HD + 8 * LPK * j + 8 * c + i] = acc[hh][8 * j + i];
    }
    if (lane == 0) {
#pragma unroll
        for (int hh = 0; hh < G; ++hh) {
            lds_m[wave][hh] = m_run[hh];
            lds_l[wave][hh] = l_run[hh];
        }
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

    // ---- publish, take a ticket; the last split of the pair merges all partials
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t t = __hip_atomic_fetch_add(a.tickets + pair, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (t == (uint32_t)(n_act - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    if (tid == 0) __hip_atomic_store(a.tickets + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

    // per-head global max / weights / denominator; weights in LDS [G][n_act]
    float* wts = lds;  // n_act <= max_splits <= 256
    const float2* ml = a.part_ml + (size_t)pair * a.max_splits * G;
    for (int hh = wave; hh < G; hh += 4) {
        float mloc = kNegInf;
        for (int t = lane; t < n_act; t += 64) mloc = fmaxf(mloc, ml[t * G + hh].x);
        const float M = wave_max(mloc);
        float lsum = 0.0f;
        for (int t = lane; t < n_act; t += 64) {
            const float2 v = ml[t * G + hh];
            const float w = exp2f(v.x - M);
            wts[hh * 256 + t] = w;
            lsum += v.y * w;
        }
        lsum = wave_sum(lsum);
        if (lane == 0) s_L[hh] = lsum;
    }
    __syncthreads();
    // each thread owns 4 consecutive outputs and streams the splits 16 at a time
    const float4* pob4 = reinterpret_cast<const float4*>(a.part_o + (size_t)pair * a.max_splits * (G * HD));
    constexpr int STRIDE4 = G * HD / 4;
    for (int e4 = tid; e4 < STRIDE4; e4 += 256) {
        const int hh = (4 * e4) / HD;
        const float* wh = wts + hh * 256;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        int t = 0;
        for (; t + 16 <= n_act; t += 16) {
            float4 v[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) v[u] = pob4[(size_t)(t + u) * STRIDE4 + e4];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const float w = wh[t + u];
                o.x = fmaf(w, v[u].x, o.x);
                o.y = fmaf(w, v[u].y, o.y);
                o.z = fmaf(w, v[u].z, o.z);
                o.w = fmaf(w, v[u].w, o.w);
            }
        }
        for (; t < n_act; ++t) {
            const float4 v = pob4[(size_t)t * STRIDE4 + e4];
            const float w = wh[t];
            o.x = fmaf(w, v.x, o.x);
            o.y = fmaf(w, v.y, o.y);
            o.z = fmaf(w, v.z, o.z);
            o.w = fmaf(w, v.w, o.w);
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
    if (((uintptr_t)k_cache | (uintptr_t)v_cache) % 16 || ((uintptr_t)q % 4) ||
        (seq_stride * esz) % 16) {
        set_error("k_cache/v_cache and seq_stride*elem_size must be 16-byte aligned");
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
