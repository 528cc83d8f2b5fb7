// KV-cache write for gfx950: k <- RoPE(RMSNorm(srq(k)) * gain), v <- RMSNorm(srq(v)),
// stored at rows start_pos.. of the [pos][kvH][hd] caches (f16, or f32).
//
// Reference semantics: kvnorm (gemma4_150/kernels_dsl.py:573-618; one token, f32 in)
// and kvnorm_b (:1789-1834; S tokens, f16 in, srq of the inputs with the k_out/v_out
// scales, RoPE by absolute position). One workgroup per (token, kv head); each
// thread owns one RoPE pair (d, d + hd/2) of k and of v.
#include "common.hpp"

namespace g4a {

struct KvArgs {
    const void* k;
    const void* v;
    const float* k_gain;
    const float* rcos;
    const float* rsin;
    void* kc;
    void* vc;
    int start_pos, n_kv_heads, v_norm;
    float k_in_q, v_in_q, eps;
};

__device__ __forceinline__ float ld(const float* p) { return *p; }
__device__ __forceinline__ float ld(const half_t* p) { return (float)*p; }

template <int HD, typename IT, typename CT>
__global__ __launch_bounds__(HD / 2) void kv_write_kernel(KvArgs a) {
    constexpr int HALF = HD / 2, NW = HALF / 64;
    __shared__ float red[2 * NW];
    const int t = threadIdx.x, s = blockIdx.x, kh = blockIdx.y;
    const size_t row = ((size_t)s * a.n_kv_heads + kh) * HD;
    const IT* kin = reinterpret_cast<const IT*>(a.k) + row;
    const IT* vin = reinterpret_cast<const IT*>(a.v) + row;
    // raw values: kv_pair_prep applies srq once its own operand loads are out (written as
    // srq(ld(..)) here, each load waited behind the previous one's zero-scale branch)
    float k0 = ld(kin + t), k1 = ld(kin + t + HALF), v0 = ld(vin + t), v1 = ld(vin + t + HALF);

    kv_pair_prep<HD>(k0, k1, v0, v1, a.k_gain, a.rcos ? a.rcos + (size_t)s * HALF : nullptr,
                     a.rsin ? a.rsin + (size_t)s * HALF : nullptr, a.v_norm != 0, a.eps, a.k_in_q, a.v_in_q,
                     red, t);
    const size_t crow = ((size_t)(a.start_pos + s) * a.n_kv_heads + kh) * HD;
    CT* kc = reinterpret_cast<CT*>(a.kc) + crow;
    CT* vc = reinterpret_cast<CT*>(a.vc) + crow;
    store_elem(kc + t, k0);
    store_elem(kc + t + HALF, k1);
    store_elem(vc + t, v0);
    store_elem(vc + t + HALF, v1);
}

typedef void (*kv_fn)(KvArgs);

template <int HD>
static kv_fn pick(bool in16, bool c32) {
    if (in16) return c32 ? kv_write_kernel<HD, half_t, float> : kv_write_kernel<HD, half_t, half_t>;
    return c32 ? kv_write_kernel<HD, float, float> : kv_write_kernel<HD, float, half_t>;
}

}  // namespace g4a

using namespace g4a;

extern "C" int g4a_kv_write(const g4a_cfg* cfg, int S, int start_pos, const void* k, const void* v,
                            float k_in_q, float v_in_q, const float* k_gain, const float* rope_cos,
                            const float* rope_sin, void* k_cache, void* v_cache, void* stream) {
    if (!check_cfg(cfg, false)) return G4A_EINVAL;
    if (S <= 0 || start_pos < 0) {
        set_error("S (%d) must be positive and start_pos (%d) non-negative", S, start_pos);
        return G4A_EINVAL;
    }
    if (!k || !v || !k_cache || !v_cache) {
        set_error("k, v, k_cache and v_cache must be non-NULL");
        return G4A_EINVAL;
    }
    if ((rope_cos == nullptr) != (rope_sin == nullptr)) {
        set_error("rope_cos and rope_sin must both be given or both be NULL");
        return G4A_EINVAL;
    }
    if (!(k_in_q >= 0.0f) || !(v_in_q >= 0.0f)) {
        set_error("k_in_q/v_in_q must be >= 0");
        return G4A_EINVAL;
    }
    const int HD = (int)cfg->head_dim;
    if (HD != 256 && HD != 512) {
        set_error("head_dim %d not supported (256 or 512)", HD);
        return G4A_EUNSUPPORTED;
    }
    if ((int64_t)S * cfg->n_kv_heads > 0x7fffffff || cfg->n_kv_heads > 65535) {
        set_error("S*n_kv_heads too large");
        return G4A_EINVAL;
    }
    const bool in16 = (cfg->flags & G4A_IN_F16) != 0, c32 = (cfg->flags & G4A_KV_F32) != 0;
    KvArgs a;
    a.k = k;
    a.v = v;
    a.k_gain = k_gain;
    a.rcos = rope_cos;
    a.rsin = rope_sin;
    a.kc = k_cache;
    a.vc = v_cache;
    a.start_pos = start_pos;
    a.n_kv_heads = (int)cfg->n_kv_heads;
    a.v_norm = (cfg->flags & G4A_NO_V_NORM) ? 0 : 1;
    a.k_in_q = k_in_q;
    a.v_in_q = v_in_q;
    a.eps = cfg->eps;
    kv_fn fn = HD == 256 ? pick<256>(in16, c32) : pick<512>(in16, c32);
    dim3 grid(S, cfg->n_kv_heads);
    hipLaunchKernelGGL(fn, grid, dim3(HD / 2), 0, (hipStream_t)stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "kv_write launch");
    return G4A_OK;
}
