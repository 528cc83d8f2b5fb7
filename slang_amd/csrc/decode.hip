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
//    A batch of several sequences runs as one work list of equal-length splits over all
//    of them (see list_chunk), so ragged lengths do not leave long splits running alone.
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
//  * Waves merge through LDS. Splits merge in a second, wide kernel (decode_merge_kernel,
//    decode_merge_list_kernel for a work list):
//    the kernel boundary publishes the partials, so no workgroup pays a cache-writeback
//    fence or a ticket round trip, and the merge of one (sequence, kv head) is spread over
//    HD/16 workgroups whose threads load all of their splits in one batch. (A last-arriver
//    merge inside this kernel, as attn_101 does, measured 2-4x slower on MI355X: its
//    agent-scope release has to write back the XCD's L2 and the merger then walks every
//    partial serially.)
// Scores are in the log2 domain (q carries scale*log2 e), so the softmax uses exp2.
#include <mutex>

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
    float2* part_ml;    // [slots][G] (m, l); slot = pair * max_splits + split, or the unit
    float* part_o;      // [slots][G][HD]
    int n_q_heads, n_kv_heads, window, max_splits, chunk;
    float scale_log2, eps, out_q;
    // work list (several sequences): list_target > 0 spreads all active keys over about
    // list_target units of equal length (>= chunk keys, <= chunk_cap), one workgroup each
    int n_seq, list_target, chunk_cap, list_units;  // list_units: the grid, units past it never run
    int fixed_len;  // key_len == NULL: every sequence has fixed_len keys (no device read)
    int2* list_tab;  // work list: (first unit, splits) per (sequence, kv head), written by split 0
    // fused KV write (g4a_decode_kv): k_new != NULL gives each sequence's raw k/v row
    // [n_seq][kvH][HD] for position key_len - 1, prepared and stored by the workgroup
    // whose split holds that key
    const float* k_new;
    const float* v_new;
    const float* k_gain;
    void* kc_out;
    void* vc_out;
    float k_in_q, v_in_q;
    int v_norm;
};

template <int HD, int G>
struct DecodeShape {
    static constexpr int KSTEPS = HD / 32;         // score MFMA k-steps per 16-key block
    static constexpr int NDT = HD / 16;            // 16-dim output tiles
    static constexpr int VLANES = HD / 8;          // lanes per V row (8 dims, 16 B each)
    static constexpr int VROWS = 64 / VLANES;      // V rows per load instruction
    static constexpr int VLOADS = 16 / VROWS;      // V load instructions per block
    static constexpr int VSTR = HD + 16;           // LDS V row stride (halves): tr reads conflict-free
    static constexpr int KSTR = HD + 8;            // LDS K row stride (halves): A-operand reads conflict-free
    static constexpr int K_HALVES = 4 * 16 * KSTR; // per-wave K blocks (whole-row K loads)
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
    static __device__ __forceinline__ raw load(rsrc_t r, int off) { return raw{bload_h8_nt(r, off)}; }
    static __device__ __forceinline__ raw lds(const half_t* p) { return raw{*reinterpret_cast<const half8*>(p)}; }
    static __device__ __forceinline__ float4v dot(const raw& k, half8 q, float4v c) { return mfma16x32(k.h, q, c); }
};
template <>
struct KOp<float> {
    struct raw { float8v f; };
    static __device__ __forceinline__ raw load(rsrc_t r, int off) { return raw{bload_f8_nt(r, off)}; }
    static __device__ __forceinline__ raw lds(const float* p) {
        const float4v a = *reinterpret_cast<const float4v*>(p), b = *reinterpret_cast<const float4v*>(p + 4);
        return raw{float8v{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]}};
    }
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
    static __device__ __forceinline__ half8 load(rsrc_t r, int off) { return bload_h8_nt(r, off); }
    static __device__ __forceinline__ half8 h(half8 v) { return v; }
};
template <>
struct VOp<float> {
    typedef float8v raw;
    static __device__ __forceinline__ float8v load(rsrc_t r, int off) { return bload_f8_nt(r, off); }
    static __device__ __forceinline__ half8 h(float8v v) { return __builtin_convertvector(v, half8); }
};

// lane n of each 16-lane row reads lane n+N of the same row
template <int N>
__device__ __forceinline__ float dpp_row_shl(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x100 + N, 0xF, 0xF, false));
}

// keys of sequence s: from the device array, or the host-given length when there is none
// (a batch-1 decode knows its position on the host, as the reference's params do)
__device__ __forceinline__ int seq_len(const DecodeArgs& a, int s) { return a.key_len ? a.key_len[s] : a.fixed_len; }

// Keys attended by sequence b and how they are split: active keys [lo, hi), split c covers
// [lo + c*chunk, min(lo + (c+1)*chunk, hi)); split c is live when c*chunk < hi - lo. No
// division on the common path: the host's chunk fits max_splits splits of max_key_len keys;
// only a key_len above max_key_len widens the chunk so the live splits still fit.
struct SplitPlan {
    int lo, hi, active, chunk;
};
__device__ __forceinline__ SplitPlan split_plan(const DecodeArgs& a, int b) {
    SplitPlan p;
    p.hi = seq_len(a, b);
    p.lo = (a.window > 0 && p.hi > a.window) ? p.hi - a.window : 0;
    p.active = p.hi - p.lo;
    p.chunk = a.chunk;
    if (p.active > a.max_splits * a.chunk)
        p.chunk = (((p.active + a.max_splits - 1) / a.max_splits) + 15) & ~15;
    return p;
}

// ---- work list over several sequences. Per-sequence splits leave the grid as ragged as
// the batch: at 16 sequences of 1K..32K keys, 2048-key splits give ~340 live workgroups of
// unequal length on 256 CUs, and the short ones finish early while the long ones cannot
// keep enough bytes in flight. Instead every workgroup computes one plan from key_len:
// chunk = ceil(sum of active keys x kvH / list_target) (a multiple of 16), sequence b gets
// ceil(active_b / chunk) splits per kv head, and the units (sequence, kv head, split) are
// numbered in that order, unit L on workgroup L. The host sizes the grid to
// list_target + pairs, which bounds the unit count, and list_target to what stays
// resident, so all units run at once and end together.
__device__ __forceinline__ int active_keys(const DecodeArgs& a, int T) {
    return T <= 0 ? 0 : (a.window > 0 && T > a.window) ? a.window : T;
}
__device__ __forceinline__ int ceil_div(int x, int d) { return x / d + (x % d != 0); }

// chunk of the plan; act0 returns this lane's sequence of the first 64 (its active keys),
// so a batch of up to 64 sequences reads key_len once
__device__ __forceinline__ int list_chunk(const DecodeArgs& a, int& act0) {
    const int lane = threadIdx.x & 63;
    unsigned long long tot = 0;
    act0 = 0;
    for (int s0 = 0; s0 < a.n_seq; s0 += 64) {
        const int s = s0 + lane;
        const int act = s < a.n_seq ? active_keys(a, seq_len(a, s)) : 0;
        if (s0 == 0) act0 = act;
        tot += (unsigned)act;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) tot += __shfl_xor(tot, d);
    unsigned long long c = (tot * (unsigned)a.n_kv_heads + a.list_target - 1) / (unsigned)a.list_target;
    c = (c + 15) & ~15ull;
    c = c < (unsigned)a.chunk ? (unsigned)a.chunk : c;
    c = c > (unsigned)a.chunk_cap ? (unsigned)a.chunk_cap : c;
    return __builtin_amdgcn_readfirstlane((int)c);
}

__device__ __forceinline__ int list_active(const DecodeArgs& a, int s0, int act0, int n) {
    const int s = s0 + (threadIdx.x & 63);
    return s0 == 0 ? (s < n ? act0 : 0) : (s < n ? active_keys(a, seq_len(a, s)) : 0);
}

struct ListUnit {
    int b, kh, ci, splits;
};
// the unit of workgroup L (b = -1: past the last unit)
__device__ __forceinline__ ListUnit list_unit(const DecodeArgs& a, int chunk, int act0, int L) {
    int base = 0;  // units of the sequences before this group of 64
    for (int s0 = 0; s0 < a.n_seq; s0 += 64) {
        const int sp = ceil_div(list_active(a, s0, act0, a.n_seq), chunk);
        const int incl = wave_prefix_sum(sp * a.n_kv_heads);
        const unsigned long long past = __ballot(base + incl > L);
        if (past) {
            const int j = __builtin_ctzll(past);
            const int splits = __builtin_amdgcn_readlane(sp, j);
            const int r = L - (base + __builtin_amdgcn_readlane(incl, j) - splits * a.n_kv_heads);
            return ListUnit{s0 + j, r / splits, r % splits, splits};
        }
        base += __builtin_amdgcn_readlane(incl, 63);
    }
    return ListUnit{-1, 0, 0, 0};
}
// QP consecutive f32 (QP = 2 or 4) from a buffer
template <int QP>
__device__ __forceinline__ void bload_q(rsrc_t r, int off, float (&x)[QP]) {
    if constexpr (QP == 2) {
        const float2 v = bload_f32x2(r, off);
        x[0] = v.x;
        x[1] = v.y;
    } else {
        const float4v v = bload_f32x4(r, off);
#pragma unroll
        for (int e = 0; e < QP; ++e) x[e] = v[e];
    }
}

// hd 256 with f16 caches fits two waves per SIMD (two workgroups per CU, which the work
// list's resident count assumes); the attribute holds the allocator to that.
// LIST: the unit comes from the work-list plan (several sequences); KVW: the fused KV write
// of g4a_decode_kv. Both are template switches so the plain single-sequence kernel carries
// neither (their code measured 0.2 us on the latency-bound T 4096 call).
template <int HD, int G, typename KVT, bool LIST, bool KVW>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(HD == 256 && sizeof(KVT) == 2 ? 2 : 1)))
void decode_kernel(DecodeArgs a) {
    using Sh = DecodeShape<HD, G>;
    constexpr int KSTEPS = Sh::KSTEPS, NDT = Sh::NDT, VLANES = Sh::VLANES, VROWS = Sh::VROWS;
    constexpr int VLOADS = Sh::VLOADS, VSTR = Sh::VSTR, QSTR = Sh::QSTR;
    constexpr int ESZ = (int)sizeof(KVT);
    using KO = KOp<KVT>;
    using VO = VOp<KVT>;
    typedef typename KO::raw kraw_t;
    typedef typename VO::raw vraw_t;
    // f16 caches: K rows are loaded whole, as V rows are (two 512-byte rows or one 1 KiB row
    // per instruction), and staged in a per-wave LDS block from which the MFMA A operands are
    // read. Loaded straight in the A layout, each instruction took 64 bytes from each of 16
    // rows; a read-only kernel over config 4's geometry streamed 6.9 TB/s with whole rows
    // against 6.4 TB/s with that pattern. (hd 512: 134 KiB of LDS, one workgroup a CU as
    // its registers allow anyway.)
    constexpr bool KROW = sizeof(KVT) == 2;
    constexpr int KSTR = Sh::KSTR;
    constexpr int ARENA = KROW && (Sh::V_HALVES + Sh::K_HALVES) * 2 > Sh::LDS_BYTES
                              ? (Sh::V_HALVES + Sh::K_HALVES) * 2 : Sh::LDS_BYTES;

    // one LDS arena, reused: q rows (prologue) -> V (and K) blocks (main loop) -> partials (merges)
    __shared__ __attribute__((aligned(16))) char arena[ARENA];
    half_t* sQ = reinterpret_cast<half_t*>(arena);
    half_t* sV = reinterpret_cast<half_t*>(arena);
    float* lds = reinterpret_cast<float*>(arena);
    __shared__ float lds_m[4][G], lds_l[4][G];
    __shared__ __attribute__((aligned(16))) KVT sKn[KVW ? HD : 8], sVn[KVW ? HD : 8];  // KVW: the new row
    __shared__ float kv_red[2 * (HD / 128)];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
    const int n = lane & 15, g = lane >> 4;
    int ci, kh, b;
    SplitPlan sp;
    size_t slot;  // partial slot of this workgroup
    if constexpr (LIST) {
        int act0;
        const int chunk = list_chunk(a, act0);
        const ListUnit u = list_unit(a, chunk, act0, blockIdx.x);
        if (u.b < 0) return;  // past the last unit
        b = u.b, kh = u.kh, ci = u.ci;
        // split 0 of each (sequence, kv head) tells the merge where its units are, so the
        // merge needs no plan of its own (a pair without keys has no unit and no entry)
        if (ci == 0 && tid == 0) a.list_tab[b * a.n_kv_heads + kh] = make_int2((int)blockIdx.x, u.splits);
        sp.hi = seq_len(a, b);
        sp.lo = (a.window > 0 && sp.hi > a.window) ? sp.hi - a.window : 0;
        sp.active = sp.hi - sp.lo;
        sp.chunk = chunk;
        slot = blockIdx.x;
    } else {
        ci = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
        sp = split_plan(a, b);  // scalar load of key_len, issued first
        slot = (size_t)(b * a.n_kv_heads + kh) * a.max_splits + ci;
    }
    float* outp = a.out + ((size_t)b * a.n_q_heads + (size_t)kh * G) * HD;

    // ---- q operand loads: they depend on nothing but the sequence and kv head.
    // Wave w prepares heads w, w+4 (a head >= G reads past the q range: zeros, no traffic).
    constexpr int QP = HD / 128;          // elements per lane in each half of a head row
    constexpr int NQH = (G + 3) / 4;      // heads per wave
    const int d0 = QP * lane;             // this lane: dims d0.. and d0+HD/2..
    const rsrc_t rq = make_rsrc(a.q + ((size_t)b * a.n_q_heads + (size_t)kh * G) * HD, G * HD * 4);
    const rsrc_t rg = make_rsrc(a.q_gain, a.q_gain ? HD * 4 : 0);
    const rsrc_t rc = make_rsrc(a.rcos ? a.rcos + (size_t)b * (HD / 2) : nullptr, a.rcos ? HD * 2 : 0);
    const rsrc_t rs = make_rsrc(a.rsin ? a.rsin + (size_t)b * (HD / 2) : nullptr, a.rsin ? HD * 2 : 0);
    float qx[NQH][2][QP], qgv[2][QP], qcv[QP], qsv[QP];
#pragma unroll
    for (int j = 0; j < NQH; ++j) {
        bload_q<QP>(rq, ((wave + 4 * j) * HD + d0) * 4, qx[j][0]);
        bload_q<QP>(rq, ((wave + 4 * j) * HD + HD / 2 + d0) * 4, qx[j][1]);
    }
    bload_q<QP>(rg, d0 * 4, qgv[0]);
    bload_q<QP>(rg, (HD / 2 + d0) * 4, qgv[1]);
    bload_q<QP>(rc, d0 * 4, qcv);
    bload_q<QP>(rs, d0 * 4, qsv);

    // ---- attended keys and this workgroup's split. With one split slot (no merge kernel)
    // this workgroup writes `out`; otherwise every slot gets a partial, and a slot past the
    // live splits a weightless (m = -inf, l = 0) marker, so the merge needs no key count.
    const bool single = a.max_splits == 1;
    if (ci * sp.chunk >= sp.active) {
        if (single) {
            for (int e = tid; e < G * HD; e += 256) outp[e] = 0.0f;  // no keys: zeros
        } else if (tid < G) {
            a.part_ml[slot * G + tid] = make_float2(kNegInf, 0.0f);
        }
        return;
    }
    const int k0 = sp.lo + ci * sp.chunk;
    const int k1 = min(k0 + sp.chunk, sp.hi);

    // ---- fused KV write: this workgroup's split holds the new key p = key_len - 1; its raw
    // k/v loads go out before the first block's, the row is prepared with the q prologue
    constexpr int HALF = HD / 2;
    const int p_new = sp.hi - 1;
    const bool owns_new = KVW && p_new >= k0 && p_new < k1;  // workgroup-uniform
    float nk0 = 0.0f, nk1 = 0.0f, nv0 = 0.0f, nv1 = 0.0f;
    KvPairOps nops{1.0f, 1.0f, 1.0f, 0.0f};
    if (owns_new) {  // with the raw row, ahead of the block loads (which they would wait behind)
        nops = kv_pair_ops<HD>(a.k_gain, a.rcos ? a.rcos + (size_t)b * HALF : nullptr,
                               a.rsin ? a.rsin + (size_t)b * HALF : nullptr, tid);
    }
    if (owns_new && tid < HALF) {
        const size_t ro = ((size_t)b * a.n_kv_heads + kh) * HD;
        // raw values: kv_pair_prep applies srq (a zero-scale branch here would wait for
        // each load before issuing the next and the block loads)
        nk0 = a.k_new[ro + tid];
        nk1 = a.k_new[ro + tid + HALF];
        nv0 = a.v_new[ro + tid];
        nv1 = a.v_new[ro + tid + HALF];
    }

    // ---- block loads through buffer resources over rows [k0, k1) of this kv head: rows
    // past k1 read as zeros without memory traffic, so no index is clamped. K in the MFMA
    // A layout (lane n,g: key n, dims 32s+8g..), V rows of VLANES lanes.
    const size_t rstride = (size_t)a.n_kv_heads * HD;  // elements per cache row
    const int rsb = (int)(rstride * ESZ);               // bytes per cache row
    const uint32_t range = (uint32_t)(k1 - k0) * (uint32_t)rsb;
    const size_t row0 = (size_t)b * a.seq_stride + (size_t)k0 * rstride + (size_t)kh * HD;
    const rsrc_t rk = make_rsrc(reinterpret_cast<const KVT*>(a.kc) + row0, range);
    const rsrc_t rv = make_rsrc(reinterpret_cast<const KVT*>(a.vc) + row0, range);
    const int vrow = lane / VLANES;
    const int koff = n * rsb + 8 * g * ESZ, voff = vrow * rsb + 8 * (lane % VLANES) * ESZ;
    kraw_t kr[KROW ? 1 : KSTEPS];
    half8 krow[KROW ? VLOADS : 1];
    vraw_t vr[VLOADS];
    auto load_block = [&](int blk) {
        const int r = (blk - k0) * rsb;
        if constexpr (KROW) {
#pragma unroll
            for (int i = 0; i < VLOADS; ++i) krow[i] = bload_h8_nt(rk, r + VROWS * i * rsb + voff);
        } else {
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) kr[s] = KO::load(rk, r + koff + 32 * s * ESZ);
        }
#pragma unroll
        for (int i = 0; i < VLOADS; ++i) vr[i] = VO::load(rv, r + VROWS * i * rsb + voff);
    };
    int blk = k0 + wave * 16;
    // in flight during the q prologue. Unconditional: a block past k1 reads zeros without
    // memory traffic. Under a branch, the join left the compiler unsure how many loads
    // followed q's, so the prologue waited for the block's loads too (vmcnt(4), not 20).
    load_block(blk);

    // ---- q prologue: RMSNorm*gain, RoPE, scale*log2 e, split into f16 high/low rows of
    // the B operand, staged in LDS.
    if (!a.rcos) {
#pragma unroll
        for (int e = 0; e < QP; ++e) {
            qcv[e] = 1.0f;
            qsv[e] = 0.0f;
        }
    }
#pragma unroll
    for (int j = 0; j < NQH; ++j) {
        const int hh = wave + 4 * j;
        if (hh >= G) break;
        float x[2][QP];
#pragma unroll
        for (int e = 0; e < QP; ++e) {
            x[0][e] = qx[j][0][e];
            x[1][e] = qx[j][1][e];
        }
        if (a.q_gain) {
            float ss = 0.0f;
#pragma unroll
            for (int e = 0; e < QP; ++e) ss += x[0][e] * x[0][e] + x[1][e] * x[1][e];
            const float rsq = 1.0f / sqrtf(wave_sum(ss) / (float)HD + a.eps);  // attn_101's q * nscale * w
#pragma unroll
            for (int e = 0; e < QP; ++e) {
                x[0][e] = x[0][e] * rsq * qgv[0][e];
                x[1][e] = x[1][e] * rsq * qgv[1][e];
            }
        }
#pragma unroll
        for (int e = 0; e < QP; ++e) {
            const float x0 = x[0][e], x1 = x[1][e];
            // pinned: the high part and the low part's subtrahend are one rounding of one value
            const float r0 = pin((x0 * qcv[e] - x1 * qsv[e]) * a.scale_log2);
            const float r1 = pin((x1 * qcv[e] + x0 * qsv[e]) * a.scale_log2);
            const half_t h0 = (half_t)r0, h1 = (half_t)r1;
            sQ[hh * QSTR + d0 + e] = h0;
            sQ[hh * QSTR + HD / 2 + d0 + e] = h1;
            sQ[(G + hh) * QSTR + d0 + e] = (half_t)(r0 - (float)h0);
            sQ[(G + hh) * QSTR + HD / 2 + d0 + e] = (half_t)(r1 - (float)h1);
        }
    }
    if (owns_new) {  // every wave takes part (one barrier inside)
        kv_pair_prep<HD>(nk0, nk1, nv0, nv1, nops, a.k_gain != nullptr, a.rcos != nullptr, a.v_norm != 0, a.eps,
                         a.k_in_q, a.v_in_q, kv_red, tid);
        if (tid < HALF) {
            const size_t crow = (size_t)b * a.seq_stride + (size_t)p_new * a.n_kv_heads * HD + (size_t)kh * HD;
            KVT* kcw = reinterpret_cast<KVT*>(a.kc_out) + crow;
            KVT* vcw = reinterpret_cast<KVT*>(a.vc_out) + crow;
            store_elem(kcw + tid, nk0);
            store_elem(kcw + tid + HALF, nk1);
            store_elem(vcw + tid, nv0);
            store_elem(vcw + tid + HALF, nv1);
            sKn[tid] = (KVT)nk0;
            sKn[tid + HALF] = (KVT)nk1;
            sVn[tid] = (KVT)nv0;
            sVn[tid + HALF] = (KVT)nv1;
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
    half_t* myK = sV + Sh::V_HALVES + wave * 16 * KSTR;  // KROW only
    float m_run = kNegInf, l_run = 0.0f;  // column n (heads: n < G)
    float4v oacc[NDT];                    // O^T[16dt + 4g + i][column n]
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = float4v{0, 0, 0, 0};

    for (; blk < k1; blk += 64) {
        // the block holding the new key: its row comes from the prepared copy, whatever
        // the load (issued before the store) returned
        const bool patch = owns_new && p_new >= blk && p_new < blk + 16;  // wave-uniform
        float4v c4 = float4v{0, 0, 0, 0};
        if constexpr (KROW) {
            // K and V rows into this wave's LDS blocks (the new key's row over whatever its
            // load returned; LDS operations of one wave complete in order), the next block's
            // loads, then the K operands back in the A layout
#pragma unroll
            for (int i = 0; i < VLOADS; ++i) {
                *reinterpret_cast<half8*>(&myK[(VROWS * i + vrow) * KSTR + 8 * (lane % VLANES)]) = krow[i];
                *reinterpret_cast<half8*>(&myV[(VROWS * i + vrow) * VSTR + 8 * (lane % VLANES)]) = VO::h(vr[i]);
            }
            if (patch && lane < HD / 8) {
                half8 hk, hv;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    hk[i] = (half_t)(float)sKn[8 * lane + i];
                    hv[i] = (half_t)(float)sVn[8 * lane + i];
                }
                *reinterpret_cast<half8*>(&myK[(p_new - blk) * KSTR + 8 * lane]) = hk;
                *reinterpret_cast<half8*>(&myV[(p_new - blk) * VSTR + 8 * lane]) = hv;
            }
            if (blk + 64 < k1) load_block(blk + 64);  // next block in flight during the products
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s)
                c4 = mfma16x32(*reinterpret_cast<const half8*>(&myK[n * KSTR + 32 * s + 8 * g]), qop[s], c4);
        } else {
            if (patch && n == p_new - blk) {
#pragma unroll
                for (int s = 0; s < KSTEPS; ++s) kr[s] = KO::lds(&sKn[32 * s + 8 * g]);
            }
#pragma unroll
            for (int s = 0; s < KSTEPS; ++s) c4 = KO::dot(kr[s], qop[s], c4);
#pragma unroll
            for (int i = 0; i < VLOADS; ++i)
                *reinterpret_cast<half8*>(&myV[(VROWS * i + vrow) * VSTR + 8 * (lane % VLANES)]) = VO::h(vr[i]);
            if (patch && lane < HD / 8) {  // rounded to f16 as VO::h rounds a loaded row
                half8 hv;
#pragma unroll
                for (int i = 0; i < 8; ++i) hv[i] = (half_t)(float)sVn[8 * lane + i];
                *reinterpret_cast<half8*>(&myV[(p_new - blk) * VSTR + 8 * lane]) = hv;
            }
            if (blk + 64 < k1) load_block(blk + 64);  // next block in flight during softmax and P.V
        }
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
        // the first block of a wave starts from zero accumulators: nothing to rescale
        if (blk != k0 + wave * 16 && __any(corr != 1.0f)) {
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= corr;
        }
        l_run = l_run * corr + ps;
        m_run = m_new;
        // O^T += V^T . P^T : lane n of group g supplies V[key 4g + n/4][16dt + 4(n%4) ..]
        const half_t* vrd = myV + (4 * g + (n >> 2)) * VSTR + 4 * (n & 3);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma16x16(lds_read_tr16(vrd + 16 * dt), pb, oacc[dt]);
    }

    // ---- workgroup merge of the wave partials through LDS: one barrier, then every thread
    // owns 4 consecutive outputs of one head and weighs the 4 waves itself.
    l_run = add32(add16(l_run));
    __syncthreads();  // every wave is done with its V block: the arena takes the partials
    if (n < G) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
            *reinterpret_cast<float4v*>(&lds[(wave * G + n) * HD + 16 * dt + 4 * g]) = oacc[dt];
        if (g == 0) {
            lds_m[wave][n] = m_run;
            lds_l[wave][n] = l_run;
        }
    }
    __syncthreads();
    for (int e = 4 * tid; e < G * HD; e += 1024) {
        const int hh = e / HD;
        float mw[4], M = kNegInf;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            mw[w] = lds_m[w][hh];
            M = fmaxf(M, mw[w]);
        }
        float L = 0.0f;
        float4v o = float4v{0, 0, 0, 0};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float wt = mw[w] == kNegInf ? 0.0f : fexp2(mw[w] - M);
            L += lds_l[w][hh] * wt;
            o += *reinterpret_cast<const float4v*>(&lds[w * G * HD + e]) * wt;
        }
        if (single) {
            const float inv = 1.0f / L;
            float4v r;
#pragma unroll
            for (int i = 0; i < 4; ++i) r[i] = srq(o[i] * inv, a.out_q);
            *reinterpret_cast<float4v*>(outp + e) = r;
        } else {
            *reinterpret_cast<float4v*>(a.part_o + slot * (G * HD) + e) = o;
            if (e % HD == 0) a.part_ml[slot * G + hh] = make_float2(M, L);
        }
    }
}

// Merge of the split partials: out = sum_c o_c 2^(m_c - M) / sum_c l_c 2^(m_c - M), M = max_c m_c
// (the flash-decoding identity attn_101 applies in its last chunk, kernels_dsl.py:1717-1749).
// One workgroup per (64 output dims, kv head, sequence). It needs no key count: every one
// of the max_splits slots holds a partial or a weightless marker, so all loads are issued
// at entry. Thread (split group sg, dim d) reads splits sg, sg+4, .. of its output element
// (NB batches of 64; slots past max_splits read as zeros through the buffer range), thread
// t reads (m, l) of split t. A slot of weight 0 is dropped by a select, never multiplied
// in: a marker slot's o holds whatever an earlier call left there.
template <int HD, int G, int NB>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
    constexpr int E = G * HD, NU = 16 * NB;
    __shared__ float wts[256];
    __shared__ float red[4][64];
    __shared__ float s_red[4], s_red2[4];
    const int tid = threadIdx.x, lane = tid & 63, sg = tid >> 6;
    const int e = blockIdx.x * 64 + lane, hh = (blockIdx.x * 64) / HD;
    const int kh = blockIdx.y, b = blockIdx.z, pair = b * a.n_kv_heads + kh;
    const int S = a.max_splits;
    const rsrc_t ro = make_rsrc(a.part_o + (size_t)pair * S * E, (uint32_t)S * E * 4);
    const rsrc_t rml = make_rsrc(a.part_ml + (size_t)pair * S * G, (uint32_t)S * G * 8);
    float v[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) v[u] = bload_f32(ro, ((sg + 4 * u) * E + e) * 4);
    const float2 mlt = bload_f32x2(rml, (tid * G + hh) * 8);
    const float mt = tid < S ? mlt.x : kNegInf;
    const float mloc = wave_max(mt);
    if (lane == 0) s_red[sg] = mloc;
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    const float w = mt == kNegInf ? 0.0f : fexp2(mt - M);
    wts[tid] = w;
    const float lw = wave_sum(w == 0.0f ? 0.0f : w * mlt.y);
    if (lane == 0) s_red2[sg] = lw;
    __syncthreads();
    float o = 0.0f;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
        const float wc = wts[sg + 4 * u];
        o = wc != 0.0f ? fmaf(wc, v[u], o) : o;
    }
    red[sg][lane] = o;
    __syncthreads();
    if (sg == 0) {
        const float L = (s_red2[0] + s_red2[1]) + (s_red2[2] + s_red2[3]);
        const float t = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
        // L = 0 only when the sequence attends no key: defined output of zeros
        a.out[((size_t)b * a.n_q_heads + (size_t)kh * G) * HD + e] = L > 0.0f ? srq(t * (1.0f / L), a.out_q) : 0.0f;
    }
}

// The same merge over a work list: the splits of (sequence b, kv head kh) are the units
// [first, first + splits) that split 0 of the pair recorded in list_tab, every one written
// by this call. Thread (sg, dim e) folds splits sg, sg+4, .. into a running (m, l, o) eight
// loads at a time; the four split groups are combined through LDS. (The partials were just
// written from other XCDs: non-temporal loads of them measured slower.)
template <int HD, int G>
__global__ __launch_bounds__(256) void decode_merge_list_kernel(DecodeArgs a) {
    constexpr int E = G * HD;
    __shared__ float sm[4][64], sl[4][64], so[4][64];
    const int tid = threadIdx.x, lane = tid & 63, sg = tid >> 6;
    const int e = blockIdx.x * 64 + lane, hh = (blockIdx.x * 64) / HD;
    const int kh = blockIdx.y, b = blockIdx.z;
    // the units of this pair, from split 0's entry; a sequence without keys has none (and
    // its entry is whatever an earlier call left)
    const int2 ent = a.list_tab[b * a.n_kv_heads + kh];
    const bool has_keys = active_keys(a, seq_len(a, b)) > 0;
    const int u0 = ent.x;
    int splits = has_keys ? ent.y : 0;
    // only with a chunk held at chunk_cap could units fall past the grid (key lengths no
    // cache in device memory can hold): their slots were never written
    if (u0 + splits > a.list_units) splits = max(0, a.list_units - u0);
    float M = kNegInf, Ls = 0.0f, O = 0.0f;
    for (int s0 = sg; s0 < splits; s0 += 32) {
        float2 ml[8];
        float o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int s = s0 + 4 * j;
            const size_t u = (size_t)u0 + (s < splits ? s : s0);
            ml[j] = a.part_ml[u * G + hh];
            o[j] = a.part_o[u * E + e];
            if (s >= splits) ml[j].x = kNegInf;
        }
        float bm = M;
#pragma unroll
        for (int j = 0; j < 8; ++j) bm = fmaxf(bm, ml[j].x);
        const float c = M == kNegInf ? 0.0f : fexp2(M - bm);  // bm is finite: split s0 is live
        Ls *= c;
        O *= c;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float w = ml[j].x == kNegInf ? 0.0f : fexp2(ml[j].x - bm);
            Ls = w != 0.0f ? fmaf(w, ml[j].y, Ls) : Ls;
            O = w != 0.0f ? fmaf(w, o[j], O) : O;
        }
        M = bm;
    }
    sm[sg][lane] = M;
    sl[sg][lane] = Ls;
    so[sg][lane] = O;
    __syncthreads();
    if (sg == 0) {
        const float Mx = fmaxf(fmaxf(sm[0][lane], sm[1][lane]), fmaxf(sm[2][lane], sm[3][lane]));
        float L = 0.0f, t = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float w = sm[k][lane] == kNegInf ? 0.0f : fexp2(sm[k][lane] - Mx);
            L = w != 0.0f ? fmaf(w, sl[k][lane], L) : L;
            t = w != 0.0f ? fmaf(w, so[k][lane], t) : t;
        }
        // L = 0 only when the sequence attends no key: defined output of zeros
        a.out[((size_t)b * a.n_q_heads + (size_t)kh * G) * HD + e] = L > 0.0f ? srq(t * (1.0f / L), a.out_q) : 0.0f;
    }
}

// ---------------------------------------------------------------- host side
// Split policy (measured on MI355X: workgroup targets of 128-1024 and minimum chunks of
// 16-512 keys were swept on configs 2 and 4 and on the whole decode step; these won or tied)
constexpr long kDecodeTargetWgs = 512;  // workgroups the worst-case sequence is spread over
constexpr long kDecodeMinChunk = 16;    // keys per split at least (one 16-key block)

constexpr long kDecodeCus = 256;        // compute units of the MI355X

// Keys per split: spread the worst-case work (every sequence at max_key_len) over about
// kDecodeTargetWgs workgroups, never below kDecodeMinChunk keys; a chunk of 64 keys
// (every wave of the workgroup busy) is preferred as long as it still yields 128 or more
// workgroups. A grid just past a whole number of rounds of one workgroup per CU (up to a
// quarter round more) is pulled back to those rounds with longer splits: the few CUs that
// would take a second workgroup each stream twice the keys of the rest (config 5's decode,
// T 8448, kvH 2: 264 workgroups of 64 keys ran 12.3 us a call, 212 of 80 keys 10.8 us).
// At most 256 splits per sequence, chunk a multiple of the 16-key block.
static int decode_chunk(const g4a_cfg* cfg, int n_seq, int max_key_len) {
    const long pairs = (long)n_seq * cfg->n_kv_heads;
    long max_active = max_key_len;
    if (cfg->window > 0 && (long)cfg->window < max_active) max_active = cfg->window;
    const long target = kDecodeTargetWgs;
    const long min_chunk = kDecodeMinChunk;
    const long kp = max_active * pairs;
    long chunk = (kp + target - 1) / target;
    if (chunk < min_chunk) chunk = min_chunk;
    if (chunk < 64 && kp >= 128L * 64) chunk = 64;
    chunk = (chunk + 15) & ~15L;
    const long wgs = pairs * ((max_active + chunk - 1) / chunk), whole = wgs / kDecodeCus * kDecodeCus;
    if (whole > 0 && wgs > whole && wgs - whole <= kDecodeCus / 4 && whole / pairs >= 1) {
        const long s = whole / pairs;  // splits per pair within the whole rounds
        chunk = (((max_active + s - 1) / s) + 15) & ~15L;
    }
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

// The work list (several sequences whose longest needs more than one split): units are
// spread over what stays resident at once -- two 4-wave workgroups per CU on the 256 CUs
// for the hd-256 f16 kernel (its registers allow two waves per SIMD), one otherwise -- less
// one unit per pair, the most the per-pair rounding up can add.
struct ListPlan {
    int target, grid;
};
static ListPlan list_plan(const g4a_cfg* cfg, int n_seq, int max_key_len) {
    ListPlan p{0, 0};
    if (n_seq <= 1 || decode_splits(cfg, n_seq, max_key_len) <= 1) return p;
    const bool f32 = (cfg->flags & G4A_KV_F32) != 0;
    const int resident = cfg->head_dim == 256 && !f32 ? 512 : 256;
    const long pairs = (long)n_seq * cfg->n_kv_heads;
    p.target = resident - pairs > resident / 2 ? (int)(resident - pairs) : resident / 2;
    p.grid = (int)(p.target + pairs);
    return p;
}

struct WsLayout {
    size_t ml, o, tab, total;
};

// partial slots: max_splits per pair, or one per work-list unit
static WsLayout ws_layout(const g4a_cfg* cfg, int n_seq, int max_key_len) {
    const ListPlan lp = list_plan(cfg, n_seq, max_key_len);
    const size_t slots = lp.grid > 0 ? (size_t)lp.grid
                                     : (size_t)n_seq * cfg->n_kv_heads * decode_splits(cfg, n_seq, max_key_len);
    const size_t G = cfg->n_q_heads / cfg->n_kv_heads;
    auto al = [](size_t x) { return (x + 255) & ~(size_t)255; };
    WsLayout L;
    L.ml = 0;
    L.o = L.ml + al(slots * G * sizeof(float2));
    L.tab = L.o + al(slots * G * cfg->head_dim * sizeof(float));
    L.total = L.tab + (lp.grid > 0 ? (size_t)n_seq * cfg->n_kv_heads * sizeof(int2) : 0);
    return L;
}

typedef void (*decode_fn)(DecodeArgs);

template <int HD, int G, typename KVT>
static decode_fn pick_mode(bool list, bool kvw) {
    if (list) return kvw ? decode_kernel<HD, G, KVT, true, true> : decode_kernel<HD, G, KVT, true, false>;
    return kvw ? decode_kernel<HD, G, KVT, false, true> : decode_kernel<HD, G, KVT, false, false>;
}
template <int HD, int G>
static decode_fn pick_kv(bool f32, bool list, bool kvw) {
    return f32 ? pick_mode<HD, G, float>(list, kvw) : pick_mode<HD, G, half_t>(list, kvw);
}
template <int HD>
static decode_fn pick_g(int G, bool f32, bool list, bool kvw) {
    switch (G) {
        case 1: return pick_kv<HD, 1>(f32, list, kvw);
        case 2: return pick_kv<HD, 2>(f32, list, kvw);
        case 4: return pick_kv<HD, 4>(f32, list, kvw);
        case 8: return pick_kv<HD, 8>(f32, list, kvw);
    }
    return nullptr;
}
template <int HD, int G>
static decode_fn pick_merge_nb(int splits) {
    if (splits <= 64) return decode_merge_kernel<HD, G, 1>;
    if (splits <= 128) return decode_merge_kernel<HD, G, 2>;
    return decode_merge_kernel<HD, G, 4>;
}
template <int HD>
static decode_fn pick_merge_list(int G) {
    switch (G) {
        case 1: return decode_merge_list_kernel<HD, 1>;
        case 2: return decode_merge_list_kernel<HD, 2>;
        case 4: return decode_merge_list_kernel<HD, 4>;
        case 8: return decode_merge_list_kernel<HD, 8>;
    }
    return nullptr;
}
template <int HD>
static decode_fn pick_merge(int G, int splits) {
    switch (G) {
        case 1: return pick_merge_nb<HD, 1>(splits);
        case 2: return pick_merge_nb<HD, 2>(splits);
        case 4: return pick_merge_nb<HD, 4>(splits);
        case 8: return pick_merge_nb<HD, 8>(splits);
    }
    return nullptr;
}

}  // namespace g4a

using namespace g4a;

extern "C" size_t g4a_decode_ws_bytes(const g4a_cfg* cfg, int n_seq, int max_key_len) {
    if (!check_cfg(cfg, true) || n_seq <= 0 || max_key_len <= 0) return 0;
    return ws_layout(cfg, n_seq, max_key_len).total;
}

struct KvNew {
    const float* k;
    const float* v;
    const float* k_gain;
    float k_in_q, v_in_q;
};

static int decode_impl(const g4a_cfg* cfg, int n_seq, int max_key_len, const int32_t* key_len,
                       const float* q, const float* q_gain, const float* rope_cos, const float* rope_sin,
                       const void* k_cache, const void* v_cache, int64_t seq_stride, float* out, void* ws,
                       size_t ws_bytes, void* stream, const KvNew* kvn) {
    if (!check_cfg(cfg, true)) return G4A_EINVAL;
    if (n_seq <= 0 || max_key_len <= 0) {
        set_error("n_seq (%d) and max_key_len (%d) must be positive", n_seq, max_key_len);
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
    const ListPlan lp = list_plan(cfg, n_seq, max_key_len);
    const WsLayout L = ws_layout(cfg, n_seq, max_key_len);
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
    a.fixed_len = max_key_len;
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
    a.list_tab = (int2*)(w + L.tab);
    a.n_q_heads = (int)cfg->n_q_heads;
    a.n_kv_heads = (int)cfg->n_kv_heads;
    a.window = (int)cfg->window;
    const int64_t row_bytes = (int64_t)cfg->n_kv_heads * HD * (int64_t)esz;
    a.n_seq = n_seq;
    a.list_target = lp.target;
    a.list_units = lp.grid;
    if (lp.grid > 0) {
        // work list: units of at least 64 keys (every wave of a workgroup busy); a unit's
        // byte offsets stay within 32 bits
        a.max_splits = 0;
        a.chunk = 64;
        a.chunk_cap = (int)(((0x7fffffff / row_bytes) - 64) & ~15LL);
        if (a.chunk_cap < a.chunk) {
            set_error("cache rows too large for 32-bit buffer offsets");
            return G4A_EINVAL;
        }
    } else {
        a.max_splits = splits;
        a.chunk = decode_chunk(cfg, n_seq, max_key_len);
        a.chunk_cap = 0;
        if ((int64_t)(a.chunk + 64) * row_bytes > 0x7fffffff) {
            set_error("keys per split too large for 32-bit buffer offsets");
            return G4A_EINVAL;
        }
    }
    a.scale_log2 = cfg->scale * kLog2e;
    a.eps = cfg->eps;
    a.out_q = cfg->out_q;
    a.k_new = kvn ? kvn->k : nullptr;
    a.v_new = kvn ? kvn->v : nullptr;
    a.k_gain = kvn ? kvn->k_gain : nullptr;
    a.kc_out = const_cast<void*>(k_cache);
    a.vc_out = const_cast<void*>(v_cache);
    a.k_in_q = kvn ? kvn->k_in_q : 0.0f;
    a.v_in_q = kvn ? kvn->v_in_q : 0.0f;
    a.v_norm = (cfg->flags & G4A_NO_V_NORM) ? 0 : 1;
    const bool list = lp.grid > 0, kvw = kvn != nullptr;
    decode_fn fn = HD == 256 ? pick_g<256>(G, f32, list, kvw) : pick_g<512>(G, f32, list, kvw);
    if (!fn) {
        set_error("no decode kernel for group size %d", G);
        return G4A_EUNSUPPORTED;
    }
    const dim3 grid = lp.grid > 0 ? dim3(lp.grid) : dim3(splits, cfg->n_kv_heads, n_seq);
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, (hipStream_t)stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "decode launch");
    if (lp.grid > 0 || splits > 1) {
        decode_fn mf = lp.grid > 0 ? (HD == 256 ? pick_merge_list<256>(G) : pick_merge_list<512>(G))
                                   : (HD == 256 ? pick_merge<256>(G, splits) : pick_merge<512>(G, splits));
        hipLaunchKernelGGL(mf, dim3(G * HD / 64, cfg->n_kv_heads, n_seq), dim3(256), 0, (hipStream_t)stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return hip_error(e, "decode merge launch");
    }
    return G4A_OK;
}

extern "C" int g4a_decode(const g4a_cfg* cfg, int n_seq, int max_key_len, const int32_t* key_len,
                          const float* q, const float* q_gain, const float* rope_cos,
                          const float* rope_sin, const void* k_cache, const void* v_cache,
                          int64_t seq_stride, float* out, void* ws, size_t ws_bytes, void* stream) {
    return decode_impl(cfg, n_seq, max_key_len, key_len, q, q_gain, rope_cos, rope_sin, k_cache, v_cache,
                            seq_stride, out, ws, ws_bytes, stream, nullptr);
}

extern "C" int g4a_decode_kv(const g4a_cfg* cfg, int n_seq, int max_key_len, const int32_t* key_len,
                             const float* q, const float* q_gain, const float* rope_cos,
                             const float* rope_sin, const float* k_new, const float* v_new, float k_in_q,
                             float v_in_q, const float* k_gain, void* k_cache, void* v_cache,
                             int64_t seq_stride, float* out, void* ws, size_t ws_bytes, void* stream) {
    if (!k_new || !v_new) {
        set_error("k_new and v_new must be non-NULL");
        return G4A_EINVAL;
    }
    if (!(k_in_q >= 0.0f) || !(v_in_q >= 0.0f)) {
        set_error("k_in_q/v_in_q must be >= 0");
        return G4A_EINVAL;
    }
    if (cfg && (cfg->flags & G4A_IN_F16)) {
        set_error("g4a_decode_kv takes f32 k/v rows (G4A_IN_F16 not supported)");
        return G4A_EUNSUPPORTED;
    }
    if ((uintptr_t)k_new % 4 || (uintptr_t)v_new % 4 || (k_gain && (uintptr_t)k_gain % 4)) {
        set_error("k_new, v_new and k_gain must be 4-byte aligned");
        return G4A_EINVAL;
    }
    const KvNew kvn{k_new, v_new, k_gain, k_in_q, v_in_q};
    return decode_impl(cfg, n_seq, max_key_len, key_len, q, q_gain, rope_cos, rope_sin, k_cache, v_cache,
                            seq_stride, out, ws, ws_bytes, stream, &kvn);
}

// ---------------------------------------------------------------- allocation-free variant
// g4a_decode_noalloc: g4a_decode with the split partials in a file-scope device array
// instead of a caller workspace, for callers that cannot allocate (code under HIP graph
// capture, serving loops that forbid hipMalloc). Each GPU holds its own copy of the array
// from the library's load until the process ends; the host reaches it only through the
// address hipGetSymbolAddress returns on that device (the array's name in host code is a
// host-side stand-in, not a device address). The partials need no initialisation (every
// slot the merge reads is written by the same call), so nothing is cleared between calls.
// Calls that overlap on one GPU share the array and race.
namespace g4a {
constexpr size_t kDecodeScratchBytes = G4A_DECODE_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kDecodeScratchBytes];
constexpr int kMaxScratchDevices = 64;
static void* g_scratch_dev[kMaxScratchDevices];  // per device: the array's device address
static std::mutex g_scratch_mu;

// The device address of this device's scratch array, resolved once per device with that
// device current (the device of the caller's stream must be the current device).
static int decode_scratch(void** p) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_error(e, "hipGetDevice");
    if (dev < 0 || dev >= kMaxScratchDevices) {
        set_error("device %d beyond the %d devices the scratch table holds", dev, kMaxScratchDevices);
        return G4A_EINVAL;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* a = nullptr;
        e = hipGetSymbolAddress(&a, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_error(e, "hipGetSymbolAddress(scratch)");
        if (!a) {
            set_error("hipGetSymbolAddress(scratch) returned NULL");
            return G4A_EHIP;
        }
        g_scratch_dev[dev] = a;
    }
    *p = g_scratch_dev[dev];
    return G4A_OK;
}
}  // namespace g4a

extern "C" int g4a_decode_noalloc(const g4a_cfg* cfg, int n_seq, int max_key_len, const int32_t* key_len,
                                  const float* q, const float* q_gain, const float* rope_cos,
                                  const float* rope_sin, const void* k_cache, const void* v_cache,
                                  int64_t seq_stride, float* out, void* stream) {
    if (!check_cfg(cfg, true)) return G4A_EINVAL;
    if (n_seq <= 0 || max_key_len <= 0) {
        set_error("n_seq (%d) and max_key_len (%d) must be positive", n_seq, max_key_len);
        return G4A_EINVAL;
    }
    const size_t need = g4a_decode_ws_bytes(cfg, n_seq, max_key_len);
    if (need == 0 || need > kDecodeScratchBytes) {
        set_error("decode partials need %zu bytes; g4a_decode_noalloc holds at most %zu "
                  "(use g4a_decode with a workspace)", need, kDecodeScratchBytes);
        return G4A_EWORKSPACE;
    }
    void* ws = nullptr;
    const int rc = decode_scratch(&ws);
    if (rc != G4A_OK) return rc;
    return decode_impl(cfg, n_seq, max_key_len, key_len, q, q_gain, rope_cos, rope_sin, k_cache, v_cache,
                       seq_stride, out, ws, kDecodeScratchBytes, stream, nullptr);
}
