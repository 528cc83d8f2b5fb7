// Batched causal prefill attention for gfx950 on f16 MFMA (v_mfma_f32_16x16x32_f16).
//
// Reference semantics: PrefillGPU._attn_gemm (gemma4_150/prefill_gpu.py:259-313) --
// qprep_b rounds the RMSNorm'd, rotated q to f16 (kernels_dsl.py:1837-1873), scores
// are q.k (scale 1.0 for Gemma 4), smax_b masks each row to [max(0, p+1-W), p]
// (:1898-1908), P.V, attnout_b divides by the row sum and applies srq(o_in)
// (:1752-1763). attn_prefill (:1950-2098) is the fused f32 form with the same mask.
//
// MI355X design: flash attention with an online softmax instead of the reference's
// materialised [S*nH][T] score matrix. A workgroup owns one kv head and BQ = 64/G
// query positions, i.e. 64 query columns = all G heads of the GQA group x BQ
// positions, so each K/V tile staged in LDS serves every head that reads it. Each of
// the 4 waves owns 16 columns. Scores are computed transposed, S^T = K . Q^T
// (A = K tile from LDS, B = Q^T held in registers), which leaves every lane with 4
// keys of ONE query column -- exactly the B-operand layout the P.V product needs
// when it is also computed transposed, O^T = V^T . P^T. V stays row-major in LDS and
// its transposed A operand comes from ds_read_tr16_b64. K/V tiles are double
// buffered in LDS: the next tile's global loads are in flight while the current one
// is computed. Scores stay f32 in the MFMA accumulators; P is rounded to f16 only as
// the MFMA operand. Tiles wholly outside [max(0, p0+1-W), p_last] are skipped;
// boundary tiles are masked per element. Work-groups are launched longest-causal-row first.
#include "common.hpp"

namespace g4a {

struct PrefillArgs {
    const float* q;
    const float* q_gain;
    const float* rcos;
    const float* rsin;
    const void* kc;
    const void* vc;
    void* out;
    int S, start_pos, n_q_heads, n_kv_heads, window, n_qblocks;
    float scale_log2, eps, out_q;
};

#ifndef G4A_PREFILL_KT256
#define G4A_PREFILL_KT256 64
#endif
template <int HD>
struct PrefillShape {
    static constexpr int KT = HD == 512 ? 32 : G4A_PREFILL_KT256;  // keys per LDS tile
    static constexpr int KSTEPS = HD / 32;           // MFMA k-steps of the score product
    static constexpr int NKT = KT / 16;              // 16-key sub-tiles of S^T
    static constexpr int NU = KT / 32;               // 32-key k-steps of the P.V product
    static constexpr int NDT = HD / 16;              // 16-dim tiles of O^T
    static constexpr int KS = HD + 8;                // K row stride (halves): A reads conflict-free
    static constexpr int VS = HD + 16;               // V row stride (halves): transpose reads conflict-free
    static constexpr int CH = HD / 8;                // 16 B chunks per row
    static constexpr int PER = KT * CH / 256;        // chunks of K (and of V) per thread per tile
    static constexpr int STAGE = KT * KS + KT * VS;  // halves per pipeline stage
};

__device__ __forceinline__ float4v mfma16(half8 a, half8 b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// 4 halves of a row-major LDS tile transposed across each 16-lane group: lane n of the
// group receives element n%4 of the 8-byte chunks supplied by lanes n/4 + 4j (j < 4).
__device__ __forceinline__ half4 lds_tr16(const half_t* p) {
    typedef short short4_ __attribute__((ext_vector_type(4)));
    const short4_ t = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_*)(p));
    return __builtin_bit_cast(half4, t);
}

// qprep_b (kernels_dsl.py:1837-1873): q RMSNorm*gain + RoPE for S*nH rows, stored f16.
// A wave handles 16 rows with the same lane layout as the prefill prologue.
template <int HD>
__global__ __launch_bounds__(256) void qprep_kernel(const float* q, const float* gain, const float* rcos,
                                                    const float* rsin, half_t* out, int rows, int n_q_heads,
                                                    float eps) {
    constexpr int KSTEPS = HD / 32;
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 16 + n;
    const bool ok = row < rows;
    const int rr = ok ? row : rows - 1;
    const int s_idx = rr / n_q_heads;
    float x[KSTEPS][8];
    prep_q_column<HD>(q + (size_t)rr * HD, gain ? gain : kOnes, rcos ? rcos + (size_t)s_idx * (HD / 2) : kOnes,
                      rsin ? rsin + (size_t)s_idx * (HD / 2) : kZeros, gain != nullptr, eps, g, x);
    if (!ok) return;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
        half8 hv;
#pragma unroll
        for (int i = 0; i < 8; ++i) hv[i] = (half_t)x[s][i];
        *reinterpret_cast<half8*>(out + (size_t)row * HD + 32 * s + 8 * g) = hv;
    }
}

template <int HD, int G, typename KVT, typename OUTT, bool HILO>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillArgs a) {
    using Sh = PrefillShape<HD>;
    constexpr int KT = Sh::KT, KSTEPS = Sh::KSTEPS, NKT = Sh::NKT, NU = Sh::NU, NDT = Sh::NDT;
    constexpr int KS = Sh::KS, VS = Sh::VS;
    constexpr int BQ = 64 / G;

    constexpr int CH = Sh::CH, PER = Sh::PER;
    __shared__ __attribute__((aligned(16))) half_t stage[2 * Sh::STAGE];  // [buf]{K[KT][KS], V[KT][VS]}

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = lane & 15, g = lane >> 4;
    const int qb = a.n_qblocks - 1 - (int)blockIdx.x;  // longest rows first
    const int kh = blockIdx.y;
    const int T_total = a.start_pos + a.S;

    // ---- this lane's query column: head hh of the group, position offset po
    const int qc = 16 * wave + n;
    const int hh = qc / BQ, po = qc % BQ;
    const int s_raw = qb * BQ + po;
    const bool col_ok = s_raw < a.S;
    const int s_idx = col_ok ? s_raw : a.S - 1;
    const int pos = a.start_pos + s_idx;
    const int h = kh * G + hh;

    // ---- q prologue: RMSNorm*gain, RoPE, f16; lane holds dims 32s + 8g + i
    half8 qf[KSTEPS], ql[HILO ? KSTEPS : 1];
    {
        float x[KSTEPS][8];
        prep_q_column<HD>(a.q + ((size_t)s_idx * a.n_q_heads + h) * HD, a.q_gain ? a.q_gain : kOnes,
                          a.rcos ? a.rcos + (size_t)s_idx * (HD / 2) : kOnes,
                          a.rsin ? a.rsin + (size_t)s_idx * (HD / 2) : kZeros, a.q_gain != nullptr, a.eps, g, x);
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const half_t hv = col_ok ? (half_t)x[s][i] : (half_t)0.0f;
                qf[s][i] = hv;
                if constexpr (HILO) ql[s][i] = col_ok ? (half_t)(x[s][i] - (float)hv) : (half_t)0.0f;
            }
    }

    // ---- key range of the workgroup and of this column
    const int p0 = a.start_pos + qb * BQ;
    const int kv_hi = min(p0 + BQ, T_total);
    const int wg_lo = (a.window > 0) ? max(0, p0 + 1 - a.window) : 0;
    const int col_lo = (a.window > 0) ? pos + 1 - a.window : 0;
    const size_t rstride = (size_t)a.n_kv_heads * HD;
    const KVT* kcb = reinterpret_cast<const KVT*>(a.kc) + (size_t)kh * HD;
    const KVT* vcb = reinterpret_cast<const KVT*>(a.vc) + (size_t)kh * HD;

    float4v oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = float4v{0, 0, 0, 0};
    float m_run = kNegInf, l_run = 0.0f;

    // ---- K/V tile staging: thread chunk r covers row (tid + 256r) / CH, chunk (tid + 256r) % CH
    half8 kst[PER], vst[PER];
    auto load_tile = [&](int t0) {
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int idx = tid + 256 * r, row = idx / CH, ch = idx % CH;
            const int key = min(t0 + row, T_total - 1);  // rows past the prompt are masked
            kst[r] = load8h(kcb + (size_t)key * rstride + 8 * ch);
            vst[r] = load8h(vcb + (size_t)key * rstride + 8 * ch);
        }
    };
    auto store_tile = [&](int buf) {
        half_t* Kb = stage + buf * Sh::STAGE;
        half_t* Vb = Kb + KT * KS;
#pragma unroll
        for (int r = 0; r < PER; ++r) {
            const int idx = tid + 256 * r, row = idx / CH, ch = idx % CH;
            *reinterpret_cast<half8*>(&Kb[row * KS + 8 * ch]) = kst[r];
            *reinterpret_cast<half8*>(&Vb[row * VS + 8 * ch]) = vst[r];
        }
    };

    const int t_first = (wg_lo / KT) * KT;
    const int ntiles = (kv_hi - t_first + KT - 1) / KT;  // >= 1: kv_hi > wg_lo
    load_tile(t_first);
    store_tile(0);
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const int t0 = t_first + it * KT, buf = it & 1;
        if (it + 1 < ntiles) load_tile(t0 + KT);  // in flight during this tile's math
        const half_t* Kb = stage + buf * Sh::STAGE;
        const half_t* Vb = Kb + KT * KS;

        // S^T = K . Q^T : sacc[kt][i] = score(key t0+16kt+4g+i, column n)
        float4v sacc[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            float4v c4 = float4v{0, 0, 0, 0};
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) {
                const half8 av = *reinterpret_cast<const half8*>(&Kb[(16 * kt + n) * KS + 32 * s + 8 * g]);
                c4 = mfma16(av, qf[s], c4);
                if constexpr (HILO) c4 = mfma16(av, ql[s], c4);
            }
            sacc[kt] = c4;
        }
        // scale (log2 domain), mask, online softmax
        float mt = kNegInf;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int key = t0 + 16 * kt + 4 * g + i;
                const bool ok = key <= pos && key >= col_lo;
                const float sv = ok ? sacc[kt][i] * a.scale_log2 : kNegInf;
                sacc[kt][i] = sv;
                mt = fmaxf(mt, sv);
            }
        mt = max32(max16(mt));
        const float m_new = fmaxf(m_run, mt);
        const float base = (m_new == kNegInf) ? 0.0f : m_new;
        const float corr = fexp2(m_run - base);
        float ps = 0.0f;
        half8 pf[NU];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p = fexp2(sacc[kt][i] - base);
                ps += p;
                pf[kt >> 1][(kt & 1) * 4 + i] = (half_t)p;
            }
        l_run = l_run * corr + ps;
        m_run = m_new;
        if (__any(corr != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= corr;
        }

        // O^T += V^T . P^T; lane n of group g supplies V[32u + 4g + n/4 (+16)][16dt + 4(n%4)..]
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const half_t* v0 = Vb + (32 * u + 4 * g + (n >> 2)) * VS + 4 * (n & 3);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) {
                const half4 lo4 = lds_tr16(v0 + 16 * dt);
                const half4 hi4 = lds_tr16(v0 + 16 * VS + 16 * dt);
                const half8 av = half8{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
                oacc[dt] = mfma16(av, pf[u], oacc[dt]);
            }
        }
        if (it + 1 < ntiles) store_tile(buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: row sum over the 4 lane groups, normalise, srq, store
    float l_tot = l_run;
    l_tot = add32(add16(l_tot));
    const float inv_l = 1.0f / l_tot;
    if (!col_ok) return;
    OUTT* orow = reinterpret_cast<OUTT*>(a.out) + ((size_t)s_idx * a.n_q_heads + h) * HD;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) store_elem(orow + 16 * dt + 4 * g + i, srq(oacc[dt][i] * inv_l, a.out_q));
}

typedef void (*prefill_fn)(PrefillArgs);

template <int HD, int G, typename KVT, typename OUTT>
static prefill_fn pick_hilo(bool hilo) {
    return hilo ? prefill_kernel<HD, G, KVT, OUTT, true> : prefill_kernel<HD, G, KVT, OUTT, false>;
}
template <int HD, int G, typename KVT>
static prefill_fn pick_out(bool out32, bool hilo) {
    return out32 ? pick_hilo<HD, G, KVT, float>(hilo) : pick_hilo<HD, G, KVT, half_t>(hilo);
}
template <int HD, int G>
static prefill_fn pick_kv(bool kv32, bool out32, bool hilo) {
    return kv32 ? pick_out<HD, G, float>(out32, hilo) : pick_out<HD, G, half_t>(out32, hilo);
}
template <int HD>
static prefill_fn pick_g(int G, bool kv32, bool out32, bool hilo) {
    switch (G) {
        case 1: return pick_kv<HD, 1>(kv32, out32, hilo);
        case 2: return pick_kv<HD, 2>(kv32, out32, hilo);
        case 4: return pick_kv<HD, 4>(kv32, out32, hilo);
        case 8: return pick_kv<HD, 8>(kv32, out32, hilo);
    }
    return nullptr;
}

}  // namespace g4a

using namespace g4a;

extern "C" size_t g4a_prefill_ws_bytes(const g4a_cfg* cfg, int S, int start_pos) {
    (void)cfg;
    (void)S;
    (void)start_pos;
    return 0;
}

extern "C" int g4a_prefill(const g4a_cfg* cfg, int S, int start_pos, const float* q,
                           const float* q_gain, const float* rope_cos, const float* rope_sin,
                           const void* k_cache, const void* v_cache, void* out, void* ws,
                           size_t ws_bytes, void* stream) {
    (void)ws;
    (void)ws_bytes;
    if (!check_cfg(cfg, true)) return G4A_EINVAL;
    if (S <= 0 || start_pos < 0) {
        set_error("S (%d) must be positive and start_pos (%d) non-negative", S, start_pos);
        return G4A_EINVAL;
    }
    if (!q || !k_cache || !v_cache || !out) {
        set_error("q, k_cache, v_cache and out must be non-NULL");
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
    if (((uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)q | (uintptr_t)out) % 16 ||
        (q_gain && (uintptr_t)q_gain % 16) || (rope_cos && ((uintptr_t)rope_cos | (uintptr_t)rope_sin) % 16)) {
        set_error("q, q_gain, rope tables, caches and out must be 16-byte aligned");
        return G4A_EINVAL;
    }
    const bool kv32 = (cfg->flags & G4A_KV_F32) != 0, out32 = (cfg->flags & G4A_OUT_F32) != 0;
    const bool hilo = (cfg->flags & G4A_Q_HILO) != 0;
    prefill_fn fn = HD == 256 ? pick_g<256>(G, kv32, out32, hilo) : pick_g<512>(G, kv32, out32, hilo);
    if (!fn) {
        set_error("no prefill kernel for group size %d", G);
        return G4A_EUNSUPPORTED;
    }
    PrefillArgs a;
    a.q = q;
    a.q_gain = q_gain;
    a.rcos = rope_cos;
    a.rsin = rope_sin;
    a.kc = k_cache;
    a.vc = v_cache;
    a.out = out;
    a.S = S;
    a.start_pos = start_pos;
    a.n_q_heads = (int)cfg->n_q_heads;
    a.n_kv_heads = (int)cfg->n_kv_heads;
    a.window = (int)cfg->window;
    const int BQ = 64 / G;
    a.n_qblocks = (S + BQ - 1) / BQ;
    a.scale_log2 = cfg->scale * kLog2e;
    a.eps = cfg->eps;
    a.out_q = cfg->out_q;
    dim3 grid(a.n_qblocks, cfg->n_kv_heads);
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, (hipStream_t)stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "prefill launch");
    return G4A_OK;
}

extern "C" int g4a_qprep(const g4a_cfg* cfg, int S, const float* q, const float* q_gain,
                         const float* rope_cos, const float* rope_sin, void* q16, void* stream) {
    if (!check_cfg(cfg, false)) return G4A_EINVAL;
    if (S <= 0 || !q || !q16) {
        set_error("S must be positive and q, q16 non-NULL");
        return G4A_EINVAL;
    }
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) {
        set_error("rope_cos and rope_sin must both be given or both be NULL");
        return G4A_EINVAL;
    }
    const int HD = (int)cfg->head_dim;
    if (HD != 256 && HD != 512) {
        set_error("head_dim %d not supported (256 or 512)", HD);
        return G4A_EUNSUPPORTED;
    }
    if (((uintptr_t)q | (uintptr_t)q16) % 16 || (q_gain && (uintptr_t)q_gain % 16) ||
        (rope_cos && ((uintptr_t)rope_cos | (uintptr_t)rope_sin) % 16)) {
        set_error("q, q_gain, rope tables and q16 must be 16-byte aligned");
        return G4A_EINVAL;
    }
    const long rows = (long)S * cfg->n_q_heads;
    if (rows > 0x7fffffffL - 64) {
        set_error("S*n_q_heads too large");
        return G4A_EINVAL;
    }
    const int blocks = (int)((rows + 63) / 64);
    auto fn = HD == 256 ? qprep_kernel<256> : qprep_kernel<512>;
    hipLaunchKernelGGL(fn, dim3(blocks), dim3(256), 0, (hipStream_t)stream, q, q_gain, rope_cos, rope_sin,
                       (half_t*)q16, (int)rows, (int)cfg->n_q_heads, cfg->eps);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "qprep launch");
    return G4A_OK;
}
