// Shared device helpers and host-side argument checking for libg4attn (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <initializer_list>

#include "../../include/g4attn.h"

namespace g4a {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float8v __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

// ---------------------------------------------------------------- host-side errors
void set_error(const char* fmt, ...);
int hip_error(hipError_t e, const char* what);
bool check_cfg(const g4a_cfg* cfg, bool need_group_le8);
// two non-NULL arrays of `bytes` bytes each that share memory
inline bool overlaps(const void* p, const void* q, size_t bytes) {
    const uintptr_t a = (uintptr_t)p, b = (uintptr_t)q;
    return p && q && a < b + bytes && b < a + bytes;
}

// ---------------------------------------------------------------- lane shuffles
// DPP row_ror:n (rotate right by n lanes within each row of 16 lanes).
template <int N>
__device__ __forceinline__ float dpp_ror(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x120 + N, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_ror<8>(x);
    x += dpp_ror<4>(x);
    x += dpp_ror<2>(x);
    x += dpp_ror<1>(x);
    return x;
}

// Cross-row exchange with gfx950's v_permlane16/32_swap (one VALU op, no LDS crossbar).
// Swapping x with itself returns the pair {x[lane], x[lane ^ 16]} (resp. ^ 32) in the same
// order in both partner lanes, so op(pair) is an exact, lane-consistent reduction step.
__device__ __forceinline__ float2 pair16(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return make_float2(__builtin_bit_cast(float, (unsigned)p[0]), __builtin_bit_cast(float, (unsigned)p[1]));
}
__device__ __forceinline__ float2 pair32(float x) {
    const unsigned u = __builtin_bit_cast(unsigned, x);
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return make_float2(__builtin_bit_cast(float, (unsigned)p[0]), __builtin_bit_cast(float, (unsigned)p[1]));
}
__device__ __forceinline__ float add16(float x) { const float2 p = pair16(x); return p.x + p.y; }
__device__ __forceinline__ float add32(float x) { const float2 p = pair32(x); return p.x + p.y; }
__device__ __forceinline__ float max16(float x) { const float2 p = pair16(x); return fmaxf(p.x, p.y); }
__device__ __forceinline__ float max32(float x) { const float2 p = pair32(x); return fmaxf(p.x, p.y); }

__device__ __forceinline__ float wave_sum(float x) { return add32(add16(row16_sum(x))); }

// Inclusive prefix sum over the 64 lanes (Hillis-Steele, six lane shifts).
__device__ __forceinline__ int wave_prefix_sum(int x) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
    x = fmaxf(x, dpp_ror<8>(x));
    x = fmaxf(x, dpp_ror<4>(x));
    x = fmaxf(x, dpp_ror<2>(x));
    x = fmaxf(x, dpp_ror<1>(x));
    return max32(max16(x));
}

// 2^x on the transcendental unit (v_exp_f32); 2^-inf = 0. Results below 2^-126 flush to
// zero, which a softmax weight relative to the running maximum can afford.
__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- buffer loads
// Raw buffer resource over [p, p + bytes): a load at a byte offset >= bytes returns zero
// and touches no memory, so a NULL operand (bytes = 0) and rows past a range need neither
// a branch nor an index clamp, and every load stays a plain vector-memory op (vmcnt only).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ float bload_f32(rsrc_t r, int off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}
__device__ __forceinline__ float2 bload_f32x2(rsrc_t r, int off) {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
}
__device__ __forceinline__ float4v bload_f32x4(rsrc_t r, int off) {
    return __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
__device__ __forceinline__ half8 bload_h8(rsrc_t r, int off) {
    return __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
// Cache policy of data read exactly once (the decode K/V stream, the decode GEMV's weight
// rows): the non-temporal bit (cpol NT). Measured against the default policy: config 4
// decode 130 -> 122-125 us, config 2 decode 8.6 -> 8.4-8.5 us, the q/k/v GEMV 4.7 -> 4.1 us.
// The prefill's K/V tiles are re-read by many query blocks through L2 and keep the default
// (NT made them 5-8 % slower).
constexpr int kCpolNT = 2;
__device__ __forceinline__ half8 bload_h8_nt(rsrc_t r, int off) {
    return __builtin_bit_cast(half8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolNT));
}
__device__ __forceinline__ float8v bload_f8_nt(rsrc_t r, int off) {
    const float4v a = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCpolNT));
    const float4v b = __builtin_bit_cast(float4v, __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, kCpolNT));
    return float8v{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}
__device__ __forceinline__ float8v bload_f8(rsrc_t r, int off) {
    const float4v a = bload_f32x4(r, off), b = bload_f32x4(r, off + 16);
    return float8v{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// ---------------------------------------------------------------- numerics
// Pin a value in a register, so the compiler can no longer fold the arithmetic that made it
// into a later conversion. A fused multiply-add-convert (v_fma_mix*_f16) rounds once, from the
// exact result, where the f32 value converted afterwards is rounded twice; near an f16 rounding
// tie the two differ by one f16 ulp. Once pinned, every conversion of x starts from the same
// f32 value: a hi/lo split sums back to x, and every kernel that rounds the same value to f16
// gets the reference's f16(f32 value) (qprep_b, kernels_dsl.py:1872-1873).
__device__ __forceinline__ float pin(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

// Static-range quantisation, identity when s == 0 (gemma4_150/reference.py:30-31).
// x / s is the IEEE quotient and rintf rounds half to even, as numpy's round does.
__device__ __forceinline__ float srq(float x, float s) {
    if (s == 0.0f) return x;
    return pin(fminf(fmaxf(rintf(x / s), -128.0f), 127.0f) * s);  // an f32 product, as the reference's
}

// gelu with the tanh approximation (reference.py:34-35), 0.5 v (1 + tanh(c (v + 0.044715 v^3)))
// with c = sqrt(2 / pi), in the equal form v / (1 + exp(-2 c (v + 0.044715 v^3))) since
// 0.5 (1 + tanh(z)) = 1 / (1 + exp(-2z)): one hardware exp2 and a division instead of tanhf,
// and no cancellation in 1 + tanh(z) where v is far below zero.
__device__ __forceinline__ float gelu_tanh16(float v) {
    const float z2 = -1.5957691216057308f * (v + 0.044715f * v * v * v);  // -2 c (..)
    return v / (1.0f + __builtin_amdgcn_exp2f(z2 * 1.4426950408889634f));
}
// GELU of v, a value already on the srq grid of step s, as the reference runners form it
// (geglu_b kernels_dsl.py:283, plegate_76 :867, gateup_74/95 :1292/:1373, plegate_b :1785):
// from the layer's 256-entry table, lut[k + 128] = f32(gelu(k s)) evaluated in float64
// (export.py:30-33), at the grid index k = clamp(round(v / s), -128, 127) -- exactly srq's
// code, since v = k s to within an f32 rounding. Without a table, or on a zero step (where
// the runners compute it too), gelu_tanh16.
__device__ __forceinline__ float gelu_srq(float v, float s, const float* lut) {
    if (!lut || s == 0.0f) return gelu_tanh16(v);
    return lut[(int)fminf(fmaxf(rintf(v / s), -128.0f), 127.0f) + 128];
}
// geglu_b's element (kernels_dsl.py:259-290) from the f16 gate and up products g, u:
// y = gelu(srq(g, gq)) * srq(u, uq), stored as its code on oq's grid (f16(y) when oq is 0)
__device__ __forceinline__ half_t geglu_code(float g, float u, float gq, float uq, float oq, const float* lut) {
    const float y = pin(gelu_srq(srq(g, gq), gq, lut) * srq(u, uq));
    return oq == 0.0f ? (half_t)y : (half_t)fminf(fmaxf(rintf(y / oq), -128.0f), 127.0f);
}

// 8 consecutive cache elements as f32, from f16 (one 16 B load) or f32 (two 16 B loads).
__device__ __forceinline__ float8v load8(const half_t* p) {
    half8 h = *reinterpret_cast<const half8*>(p);
    return __builtin_convertvector(h, float8v);
}
__device__ __forceinline__ float8v load8(const float* p) {
    float4v a = *reinterpret_cast<const float4v*>(p);
    float4v b = *reinterpret_cast<const float4v*>(p + 4);
    return float8v{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// 8 consecutive cache elements as f16 (the MFMA operand type).
__device__ __forceinline__ half8 load8h(const half_t* p) { return *reinterpret_cast<const half8*>(p); }
__device__ __forceinline__ half8 load8h(const float* p) {
    return __builtin_convertvector(load8(p), half8);
}

__device__ __forceinline__ void store_elem(half_t* p, float v) { *p = (half_t)v; }
__device__ __forceinline__ void store_elem(float* p, float v) { *p = v; }

// 4 consecutive outputs (16-byte aligned for f32, 8-byte for f16) in one store
__device__ __forceinline__ void store4(half_t* p, float4v v) {
    *reinterpret_cast<half4*>(p) = __builtin_convertvector(v, half4);
}
__device__ __forceinline__ void store4(float* p, float4v v) { *reinterpret_cast<float4v*>(p) = v; }
// srq of 4 values with one test of the step (0 = pass-through)
__device__ __forceinline__ float4v srq4(float4v x, float s) {
    if (s == 0.0f) return x;
    return float4v{srq(x[0], s), srq(x[1], s), srq(x[2], s), srq(x[3], s)};
}

// Stand-ins for absent operands, so operand loads never sit behind a null test and
// can all be issued before any arithmetic: gain 1 (used only when a norm is asked for)
// and the identity rotation cos 1 / sin 0, which leaves x exactly unchanged.
#define G4A_ONES8 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f
#define G4A_ONES64 G4A_ONES8, G4A_ONES8, G4A_ONES8, G4A_ONES8, G4A_ONES8, G4A_ONES8, G4A_ONES8, G4A_ONES8
__device__ __attribute__((aligned(16))) static const float kOnes[512] = {
    G4A_ONES64, G4A_ONES64, G4A_ONES64, G4A_ONES64, G4A_ONES64, G4A_ONES64, G4A_ONES64, G4A_ONES64};
__device__ __attribute__((aligned(16))) static const float kZeros[512] = {};

// q RMSNorm*gain then split-half RoPE for one query row, in the MFMA B-operand layout:
// the lane of k-group g holds dims 32s + 8g + i (s < hd/32, i < 8), so the RoPE partner
// d + hd/2 sits in the same lane at step s + hd/64 and the row's sum of squares needs
// only the two cross-group shuffles. Every operand is loaded before any arithmetic
// (one memory round trip). `gain` and `cr`/`sr` must be valid: kOnes / kZeros stand in
// for absent operands; `norm` says whether to normalise at all. Shared by the prefill
// and qprep kernels, whose lane layouts match, so both round the same values to f16.
template <int HD>
__device__ __forceinline__ void prep_q_column(const float* qr, const float* gain, const float* cr,
                                              const float* sr, bool norm, float eps, int g,
                                              float (&x)[HD / 32][8]) {
    constexpr int KSTEPS = HD / 32;
    float8v gv[KSTEPS], cv[KSTEPS / 2], sv[KSTEPS / 2];
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
        const float8v v = load8(qr + 32 * s + 8 * g);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[s][i] = v[i];
        gv[s] = load8(gain + 32 * s + 8 * g);
    }
#pragma unroll
    for (int s = 0; s < KSTEPS / 2; ++s) {
        cv[s] = load8(cr + 32 * s + 8 * g);
        sv[s] = load8(sr + 32 * s + 8 * g);
    }
    if (norm) {
        float ss = 0.0f;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(x[s][i], x[s][i], ss);
        ss = add32(add16(ss));
        const float rs = 1.0f / sqrtf(ss / (float)HD + eps);  // x * rs * w, as the reference kernels
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) x[s][i] = x[s][i] * rs * gv[s][i];
    }
#pragma unroll
    for (int s = 0; s < KSTEPS / 2; ++s)
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x0 = x[s][i], x1 = x[s + KSTEPS / 2][i];
            // explicit fma, and the result pinned: every user rounds the same f32 value
            x[s][i] = pin(__builtin_fmaf(x0, cv[s][i], -(x1 * sv[s][i])));
            x[s + KSTEPS / 2][i] = pin(__builtin_fmaf(x1, cv[s][i], x0 * sv[s][i]));
        }
}

// Position of workgroup L in a work list cut into 8 contiguous runs, one per XCD (the
// dispatcher deals workgroup L to XCD L % 8): XCDs x < r take `per` items, the rest per - 1.
__device__ __forceinline__ int xcd_run_index() {
    const int N = gridDim.x, L = blockIdx.x, x = L % 8, slot = L / 8;
    const int per = (N + 7) / 8, r = N - 8 * (per - 1);
    return x < r ? x * per + slot : r * per + (x - r) * (per - 1) + slot;
}

// One RoPE pair (d, d + hd/2) of a new k and v row, per thread t = d < hd/2 of the first
// hd/128 waves (kvnorm, kernels_dsl.py:573-618; kvnorm_b, :1789-1834): k <- RoPE(RMSNorm(
// srq(k)) * gain), v <- RMSNorm(srq(v)) without scale, from the raw loaded values. The sums
// of squares run per wave then over the waves in order through `red` (2 x hd/128 floats of
// LDS), so g4a_kv_write and the fused decode write identical rows. Every wave of the
// workgroup must call it (one barrier); threads t >= hd/2 pass zeros and ignore the result.
// The pair's gain and rotation operands come from kv_pair_ops, which a kernel may call
// early: loads return in issue order, so operands loaded after other traffic (the fused
// decode's K/V block) would wait for it.
struct KvPairOps {
    float g0, g1, c, sn;
};
template <int HD>
__device__ __forceinline__ KvPairOps kv_pair_ops(const float* k_gain, const float* rcos, const float* rsin, int t) {
    constexpr int HALF = HD / 2;
    const int tl = t < HALF ? t : 0;
    KvPairOps o;
    o.g0 = k_gain ? k_gain[tl] : 1.0f;
    o.g1 = k_gain ? k_gain[tl + HALF] : 1.0f;
    o.c = rcos ? rcos[tl] : 1.0f;
    o.sn = rcos ? rsin[tl] : 0.0f;
    return o;
}
template <int HD>
__device__ __forceinline__ void kv_pair_prep(float& k0, float& k1, float& v0, float& v1, const KvPairOps& o,
                                             bool has_gain, bool has_rope, bool v_norm, float eps, float k_in_q,
                                             float v_in_q, float* red, int t) {
    constexpr int HALF = HD / 2, NW = HALF / 64;
    k0 = srq(k0, k_in_q);
    k1 = srq(k1, k_in_q);
    v0 = srq(v0, v_in_q);
    v1 = srq(v1, v_in_q);
    const float sk_w = wave_sum(k0 * k0 + k1 * k1), sv_w = wave_sum(v0 * v0 + v1 * v1);
    if (t < HALF && (t & 63) == 0) {
        red[t >> 6] = sk_w;
        red[NW + (t >> 6)] = sv_w;
    }
    __syncthreads();
    if (t >= HALF) return;
    float sk = 0.0f, sv = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        sk += red[w];
        sv += red[NW + w];
    }
    if (has_gain) {
        const float rs = 1.0f / sqrtf(sk / (float)HD + eps);  // kvnorm's k * rmsk * knorm
        k0 = k0 * rs * o.g0;
        k1 = k1 * rs * o.g1;
    }
    if (has_rope) {
        // explicit fma forms: the two kernels that inline this (g4a_kv_write's and the fused
        // decode write) must not contract the rotation differently
        const float x0 = k0, x1 = k1;
        k0 = __builtin_fmaf(x0, o.c, -(x1 * o.sn));
        k1 = __builtin_fmaf(x1, o.c, x0 * o.sn);
    }
    if (v_norm) {
        const float rs = 1.0f / sqrtf(sv / (float)HD + eps);
        v0 = v0 * rs;
        v1 = v1 * rs;
    }
    // the rows are rounded to the cache type by the caller: from these f32 values
    k0 = pin(k0);
    k1 = pin(k1);
    v0 = pin(v0);
    v1 = pin(v1);
}
// The same with its operands loaded here: they load before srq (whose zero-scale branch
// waits for the raw values) and before the reduction's barrier, so they share the raw
// row's round trip.
template <int HD>
__device__ __forceinline__ void kv_pair_prep(float& k0, float& k1, float& v0, float& v1, const float* k_gain,
                                             const float* rcos, const float* rsin, bool v_norm, float eps,
                                             float k_in_q, float v_in_q, float* red, int t) {
    const KvPairOps o = kv_pair_ops<HD>(k_gain, rcos, rsin, t);
    kv_pair_prep<HD>(k0, k1, v0, v1, o, k_gain != nullptr, rcos != nullptr, v_norm, eps, k_in_q, v_in_q, red, t);
}

}  // namespace g4a
