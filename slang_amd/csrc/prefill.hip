// Batched causal prefill attention for gfx950 on f16 MFMA (v_mfma_f32_32x32x16_f16).
//
// Reference semantics: PrefillGPU._attn_gemm (gemma4_150/prefill_gpu.py:259-313) --
// qprep_b rounds the RMSNorm'd, rotated q to f16 (kernels_dsl.py:1837-1873), scores
// are q.k (scale 1.0 for Gemma 4), smax_b masks each row to [max(0, p+1-W), p]
// (:1898-1908), P.V, attnout_b divides by the row sum and applies srq(o_in)
// (:1752-1763). attn_prefill (:1950-2098) is the fused f32 form with the same mask, on
// f32 q and f32 caches.
//
// MI355X design: flash attention with an online softmax instead of the reference's
// materialised [S*nH][T] score matrix. A workgroup owns one kv head and a block of query
// columns (all G heads of the GQA group x the block's positions), so each K/V tile staged
// in LDS serves every head that reads it. Scores are computed transposed, S^T = K . Q^T
// (A = K tile from LDS, B = Q^T held in registers), which leaves every lane with keys of
// ONE query column -- exactly the B-operand layout the P.V product needs when it is also
// computed transposed, O^T = V^T . P^T. V stays row-major in LDS and its transposed A
// operand comes from ds_read_tr16_b64. K/V tiles are DMA'd straight into LDS, double
// buffered. Scores stay f32 in the MFMA accumulators; P is rounded to f16 only as the MFMA
// operand. Tiles wholly outside [max(0, p0+1-W), p_last] are skipped; boundary tiles are
// masked per element. Workgroups are launched longest-causal-row first.
//
// Precision modes: q in f16 (qprep_b's rounding point, the GEMM form), or f32-accurate as
// the f16 pair (q_hi, q_lo) (G4A_Q_HILO, attn_prefill's f32 q). f32 caches (G4A_KV_F32) are
// converted to f16 as the GEMM form's srqh_b does, and with G4A_Q_HILO (attn_prefill on its
// own f32 caches) K is kept as the f16 pair (k_hi, k_lo), so the scores are f32-accurate.
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
    // key split of long causal rows (prefill_kernel_w32): split_tiles = 0 means none;
    // otherwise a workgroup covers at most split_tiles key tiles of its query block and
    // blocks with more tiles leave partials for prefill_merge_kernel
    int split_tiles, max_pieces, pieces_per_head;
    int xcd_runs;  // prefill_kernel_w32 unsplit: 1-D grid, query blocks in contiguous runs per XCD
    int xcd_heads;  // unsplit causal: 1-D grid, kv head h on XCDs 8h/kvH .., its blocks longest first
    const half_t* q16;  // prefill_kernel_w32: q already prepared in f16 (qprep_kernel), or NULL
    const half_t* q16lo;  // ... and with G4A_Q_HILO its f16 low parts (q - f32(q16))
    int kv_row0;  // prefill_kernel_w32: first row held in kc/vc (rows below it are never read)
    const void* kclo;  // f32 caches: the f16 low parts k - f32(f16(k)) of the f16 K copy in kc
    half_t* part_o;   // [kvH][n_qblocks][max_pieces] blocks of NCOL x HD O / l in f16, in the
                      // accumulator layout [wave block][dt][j pair][lane][8] (see prefill_merge_kernel)
    float2* part_ml;  // [kvH][n_qblocks][max_pieces][128 columns] (m, l)
};

// Most a column's running maximum lags its true maximum by (log2 units): P <= 2^15 < 65504
constexpr float kMaxLag = 15.0f;

// Rows j0 .. j0 + 7 of a 32x32 accumulator tile (two 4-row groups of one lane) times inv,
// as one 16-byte f16 store: the split pieces' partial O. NT: on the non-temporal policy,
// which the hd-256 pieces take (their 12 MB of partials at S 1024, with the q rows also
// stored that way: config 3G 27.2 -> 26.5 us, 3S 25.2 -> 25.55 us) and the hd-512 ones do
// not (29 MB: 47.3 -> 49.2 us).
template <bool NT, typename ACC>
__device__ __forceinline__ void store_part8(half_t* dst, const ACC& acc, int j0, float inv) {
    half8 v;
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (half_t)(acc[j0 + i] * inv);
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<half8*>(dst));
    else *reinterpret_cast<half8*>(dst) = v;
}

// LDS operand reads issued ahead of their MFMAs in prefill_kernel_w32: score product
// (one K read per MFMA) and P.V product (two transposed V reads per MFMA); 2-8 and 3-7
// measured within +-2 % at S 1024 and S 8192
constexpr int kQkAhead = 4;
constexpr int kPvAhead = 3;
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
                                                    float eps, half_t* out_lo) {
    constexpr int KSTEPS = HD / 32;
    const int lane = threadIdx.x & 63, n = lane & 15, g = lane >> 4;
    const int row = (blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)) * 16 + n;
    const bool ok = row < rows;
    const int rr = ok ? row : rows - 1;
    const int s_idx = rr / n_q_heads;
    float x[KSTEPS][8];
    prep_q_column<HD>(q + (size_t)rr * HD, gain ? gain : kOnes, rcos ? rcos + (size_t)s_idx * (HD / 2) : kOnes,
                      rsin ? rsin + (size_t)s_idx * (HD / 2) : kZeros, gain != nullptr, eps, g, x);
    if (!ok) return;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
        half8 hv, lv;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            hv[i] = (half_t)x[s][i];
            lv[i] = (half_t)(x[s][i] - (float)hv[i]);  // the f32-accurate split of G4A_Q_HILO
        }
        // non-temporal: the attention kernel reads these rows after this kernel has ended
        // (with the pieces' partials likewise: config 3G 27.2 -> 26.5 us, 3S 25.2 -> 25.55)
        __builtin_nontemporal_store(hv, reinterpret_cast<half8*>(out + (size_t)row * HD + 32 * s + 8 * g));
        if (out_lo) *reinterpret_cast<half8*>(out_lo + (size_t)row * HD + 32 * s + 8 * g) = lv;
    }
}

// The same preparation for hd 512, one wave per row (rows of four waves a workgroup): lane l
// holds dims 8l .. 8l+7, its RoPE partner (d, d + 256) sits in lane l ^ 32. Only the hd-512
// kernels read this q, and only from here, so its sum-of-squares order (per lane, then
// across the wave) need not be prep_q_column's; the RoPE arithmetic is. Eight 16-byte loads
// a lane, against qprep_kernel's 96 for the same row share.
__global__ __launch_bounds__(256) void qprep_row512_kernel(const float* q, const float* gain, const float* rcos,
                                                         const float* rsin, half_t* out, int rows, int n_q_heads,
                                                         float eps, half_t* out_lo) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // wave-uniform
    const int s_idx = row / n_q_heads;
    float8v x = load8(q + (size_t)row * 512 + 8 * lane);
    float8v c = float8v{1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f}, sn = float8v{};
    if (rcos) {
        c = load8(rcos + (size_t)s_idx * 256 + 8 * (lane & 31));
        sn = load8(rsin + (size_t)s_idx * 256 + 8 * (lane & 31));
    }
    if (gain) {
        const float8v gv = load8(gain + 8 * lane);
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(x[i], x[i], ss);
        const float rs = 1.0f / sqrtf(wave_sum(ss) / 512.0f + eps);  // x * rs * w, as the reference kernels
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = x[i] * rs * gv[i];
    }
    half8 hv, lv;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float y = __shfl_xor(x[i], 32);
        // lane < 32: x0 = x, x1 = y; lane >= 32: x1 = x, x0 = y (prep_q_column's fma forms)
        const float r = lane < 32 ? pin(__builtin_fmaf(x[i], c[i], -(y * sn[i]))) : pin(__builtin_fmaf(x[i], c[i], y * sn[i]));
        hv[i] = (half_t)r;
        lv[i] = (half_t)(r - (float)hv[i]);
    }
    *reinterpret_cast<half8*>(out + (size_t)row * 512 + 8 * lane) = hv;
    if (out_lo) *reinterpret_cast<half8*>(out_lo + (size_t)row * 512 + 8 * lane) = lv;
}

// q to f16 (and its low parts) for S x nH rows on `stream`
static hipError_t launch_qprep(int HD, long rows, int n_q_heads, const float* q, const float* gain,
                               const float* rcos, const float* rsin, half_t* out, half_t* out_lo, float eps,
                               hipStream_t stream) {
    if (HD == 256)  // one wave (16 rows) per workgroup spreads even short prompts over every CU
        hipLaunchKernelGGL(qprep_kernel<256>, dim3((unsigned)((rows + 15) / 16)), dim3(64), 0, stream, q, gain, rcos,
                           rsin, out, (int)rows, n_q_heads, eps, out_lo);
    else
        hipLaunchKernelGGL(qprep_row512_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, stream, q, gain, rcos,
                           rsin, out, (int)rows, n_q_heads, eps, out_lo);
    return hipGetLastError();
}

// ---------------------------------------------------------------- hd 256
// prefill_kernel_w32: 32 query columns per wave (128 per workgroup: G heads x 128/G
// positions) on v_mfma_f32_32x32x16_f16, so each K or V operand read from LDS feeds a
// 32-column MFMA (16 columns would double the LDS bytes per FLOP). K/V tiles of 64 keys go straight from
// HBM into LDS (buffer_load ... lds, 16 B per lane, no staging registers), double buffered,
// one barrier per tile. LDS rows are 512 B with the 16-byte chunk c of row r stored at a
// swizzled position: c ^ (r % 32) for K, whose reads take one chunk of 32 consecutive rows,
// and c ^ vswz(r % 4) for V, whose transposed reads take 2 (16 lanes) or 4 (32 lanes)
// adjacent chunks of 4 consecutive rows: vswz = {0, 10, 12, 6} puts those rows' 32-byte
// pairs in distinct 128-byte and their 64-byte quads in distinct 256-byte bank windows.
// The running maximum of a column lags: it moves only when a score exceeds it by more than
// 2^kMaxLag, and then every column of the wave takes its own current maximum (the rescale
// of the O^T accumulators is one wave-wide pass either way), so rescales stay rare and P
// stays <= 2^kMaxLag, inside f16's range.
typedef float float16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float16v mfma32(half8 a, half8 b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int vswz(int r) { return (0x6CA0 >> (4 * (r & 3))) & 15; }

// ---- the workgroup's query block (longest causal rows first) and, with a key split, its
// piece: the work lists of the 32-column kernels (query blocks of BQ positions, KT-key tiles).
// The split grid is 1-D: the work list (kv head, block from the longest, piece) is cut into
// 8 contiguous runs, one per XCD (the dispatcher deals workgroup L to XCD L % 8), so the
// pieces of a block share one L2 for the block's q rows and each kv head's K/V is read by as
// few XCDs as the split allows: every kernel starts with cold L2s, and the first tiles of all
// workgroups arrive together. Within its kv head, piece i is found by counting through the
// blocks from the longest, each holding ceil(tiles / split_tiles) pieces: the lanes take 64
// blocks at a time (one division each, in parallel) and a prefix sum over the wave finds the
// block holding piece i; a scalar loop over the blocks would cost microseconds of issue slots.
struct PrefillUnit {
    int kh, qb, piece, n_pieces;
};
template <int BQ, int KT>
__device__ __forceinline__ PrefillUnit prefill_unit(const PrefillArgs& a, int lane) {
    const int T_total = a.start_pos + a.S;
    // key tiles of query block b: [lo(b), hi(b)) in tiles of KT keys
    auto block_tiles = [&](int b) {
        const int b0 = a.start_pos + b * BQ;
        const int hi = min(b0 + BQ, T_total), lo = a.window > 0 ? max(0, b0 + 1 - a.window) : 0;
        return (hi - lo + KT - 1) / KT;
    };
    int kh = blockIdx.y, qb = a.n_qblocks - 1 - (int)blockIdx.x, piece = 0, n_pieces = 1;
    if (a.xcd_heads) {
        // causal, unsplit: kv head kh on its own 8/kvH XCDs (the dispatcher deals workgroup L
        // to XCD L % 8), each head's blocks longest first across them
        const int L = blockIdx.x, x = L % 8, hpx = 8 / a.n_kv_heads;
        kh = x / hpx;
        qb = a.n_qblocks - 1 - ((L / 8) * hpx + x % hpx);
    }
    if (a.xcd_runs) {
        // sliding window, unsplit: a 1-D grid over (kv head, query block) in contiguous runs
        // per XCD, so neighbouring blocks -- which share most of their window's K/V tiles --
        // run on one L2 at the same time
        const int v = xcd_run_index();
        kh = v / a.n_qblocks;
        qb = v - kh * a.n_qblocks;
    }
    if (a.split_tiles > 0) {
        const int v = xcd_run_index();
        kh = v / a.pieces_per_head;
        const int i = v - kh * a.pieces_per_head;
        int base = 0;  // pieces of the blocks before this group of 64
        for (int k0 = 0; k0 < a.n_qblocks; k0 += 64) {
            const int b = a.n_qblocks - 1 - (k0 + lane);
            const int np = b >= 0 ? max(1, (block_tiles(b) + a.split_tiles - 1) / a.split_tiles) : 0;
            const int incl = wave_prefix_sum(np);
            const unsigned long long past = __ballot(base + incl > i);  // lanes whose range ends past piece i
            if (past) {
                const int L = __builtin_ctzll(past);
                qb = a.n_qblocks - 1 - (k0 + L);
                n_pieces = __builtin_amdgcn_readlane(np, L);
                piece = i - (base + __builtin_amdgcn_readlane(incl, L) - n_pieces);
                break;
            }
            base += __builtin_amdgcn_readlane(incl, 63);
        }
    }
    return PrefillUnit{kh, qb, piece, n_pieces};
}

template <int G, typename OUTT, bool HILO, bool KLO, bool SPLITK>
__global__ __launch_bounds__(256) void prefill_kernel_w32(PrefillArgs a) {
    constexpr int HD = 256, KT = 64, NCOL = 128, BQ = NCOL / G;
    constexpr int QMF = HILO ? 2 : 1;  // score MFMAs per K operand (q high, then low parts)
    constexpr int RPU = KLO ? 2 : 1;   // LDS reads per K operand (K high, then low parts)
    constexpr int MPU = QMF + (KLO ? 1 : 0);  // score MFMAs per K operand pair
    constexpr int NB = KLO ? 2 : 4;    // K operands read per batch
    constexpr int AHEAD = KLO ? 2 : kQkAhead;
    constexpr int ROWB = HD * 2;      // bytes per LDS tile row
    constexpr int TILEB = KT * ROWB;  // one K or V tile
    // [buffer][K, V]; with KLO one more tile: the K low parts of the current tile, single
    // buffered (refilled once every wave has formed its scores)
    __shared__ __attribute__((aligned(1024))) char lds[2 * 2 * TILEB + (KLO ? TILEB : 0)];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n32 = lane & 31, h = lane >> 5;
    const int T_total = a.start_pos + a.S;
    const PrefillUnit wu = prefill_unit<BQ, KT>(a, lane);
    const int kh = wu.kh, qb = wu.qb, piece = wu.piece, n_pieces = wu.n_pieces;

    // ---- key range of the workgroup [wg_lo, kv_hi) in tiles; with a key split this
    // workgroup takes tiles [t0, t1) of its query block
    const int p0 = a.start_pos + qb * BQ;
    const int kv_hi = min(p0 + BQ, T_total);
    const int wg_lo = a.window > 0 ? max(0, p0 + 1 - a.window) : 0;
    const int n_tiles = (kv_hi - wg_lo + KT - 1) / KT;
    int t0 = 0, t1 = n_tiles;
    if (a.split_tiles > 0) {
        t0 = piece * a.split_tiles;
        t1 = min(t0 + a.split_tiles, n_tiles);
    }

    // ---- this lane's query column (head hh, position offset pl) and 8-dim half h
    const int c = 32 * wave + n32;
    const int hh = c % G, pl = c / G;
    const int s_raw = qb * BQ + pl;
    const bool col_ok = s_raw < a.S;
    const int s_idx = col_ok ? s_raw : a.S - 1;
    const int pos = a.start_pos + s_idx;

    // K/V of this kv head through buffer resources: rows >= kv_hi read as zeros
    const int rowg = a.n_kv_heads * HD * 2;  // global bytes per cache row
    // (rows from kv_row0: a cache converted to f16 for this call holds only the attended rows)
    const rsrc_t rk = make_rsrc(reinterpret_cast<const half_t*>(a.kc) + (size_t)kh * HD, (uint32_t)(kv_hi - a.kv_row0) * rowg);
    const rsrc_t rv = make_rsrc(reinterpret_cast<const half_t*>(a.vc) + (size_t)kh * HD, (uint32_t)(kv_hi - a.kv_row0) * rowg);
    // wave w fills tile rows 16w .. 16w+15, two rows (1 KiB) per instruction
    auto issue = [&](int t, int buf) {
        const int kb = wg_lo + t * KT - a.kv_row0;
        char* kdst = lds + buf * 2 * TILEB;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = 16 * wave + 2 * j + h;  // tile row of this lane
            const int kvo = (kb + r) * rowg + 16 * (n32 ^ (r & 31));
            const int vvo = (kb + r) * rowg + 16 * (n32 ^ vswz(r));
            char* d = kdst + (16 * wave + 2 * j) * ROWB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)d, 16, kvo, 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(d + TILEB), 16, vvo, 0, 0, 0);
        }
    };
    // K low parts of tile t into their own stage, in K's layout (8 instructions a wave)
    const rsrc_t rkl = make_rsrc(KLO ? reinterpret_cast<const half_t*>(a.kclo) + (size_t)kh * HD : nullptr,
                                 KLO ? (uint32_t)(kv_hi - a.kv_row0) * rowg : 0u);
    auto issue_klo = [&](int t) {
        const int kb = wg_lo + t * KT - a.kv_row0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = 16 * wave + 2 * j + h;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rkl, (__attribute__((address_space(3))) void*)(lds + 4 * TILEB + (16 * wave + 2 * j) * ROWB),
                                                     16, (kb + r) * rowg + 16 * (n32 ^ (r & 31)), 0, 0, 0);
        }
    };

    // ---- q prologue: lane (column, h) holds dims 16s + 8h + i (s < 16, i < 8), the B
    // operand layout of the 32x32x16 MFMA. The arithmetic, including the order of the
    // sum of squares, is that of prep_q_column (qprep_kernel), so both round q to the
    // same f16 values: lane h holds prep_q_column's k-groups h (even s) and h + 2 (odd s).
    half8 qf[16], ql[HILO ? 16 : 1];
    // SPLITK: a launch with a key split, whose q16 comes from qprep_kernel (a template flag,
    // so each launch runs a kernel with only its own prologue and epilogue: 3S 24.95 -> 23.7 us,
    // 3G 26.5 -> 26.1 us against one kernel holding both)
    if constexpr (SPLITK) {  // q prepared by qprep_kernel for every piece of the call at once
        // Wave w DMAs the f16 q rows of its own 32 columns (two 512-byte rows per
        // instruction, chunk n32 of a row from logical chunk n32 ^ (row % 32)) into the LDS
        // stage that tile t0 + 1 takes over later, then reads them back in the B-operand
        // layout. Whole rows keep every global access a full 1 KiB run.
        const rsrc_t rq = make_rsrc(a.q16, (uint32_t)a.S * a.n_q_heads * HD * 2);
        char* qs = lds + ((t0 + 1) & 1) * 2 * TILEB;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int r = 32 * wave + 2 * j + h;  // column of the row this lane moves
            const int qo = ((qb * BQ + r / G) * a.n_q_heads + kh * G + r % G) * ROWB + 16 * (n32 ^ (r & 31));
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (__attribute__((address_space(3))) void*)(qs + (32 * wave + 2 * j) * ROWB),
                                                     16, qo, 0, 0, 0);
        }
        if (t0 < t1) issue(t0, t0 & 1);
        if (KLO && t0 < t1) issue_klo(t0);
        // the 16 q DMAs were issued before tile t0's 16 (+ 8 K low): done at vmcnt <= 16 (24)
        if (t0 >= t1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else if constexpr (KLO) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        const char* qrow = qs + c * ROWB;
#pragma unroll
        for (int s = 0; s < 16; ++s) qf[s] = *reinterpret_cast<const half8*>(qrow + 16 * ((2 * s + h) ^ n32));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // stage free for tile t0 + 1's DMA
        if constexpr (HILO) {  // the low parts straight into the operand layout
            const rsrc_t rql = make_rsrc(a.q16lo, (uint32_t)a.S * a.n_q_heads * HD * 2);
            const int qo = (s_idx * a.n_q_heads + kh * G + hh) * ROWB + 16 * h;
#pragma unroll
            for (int s = 0; s < 16; ++s) ql[s] = bload_h8(rql, qo + 32 * s);
        }
        if (!col_ok) {
#pragma unroll
            for (int s = 0; s < 16; ++s) qf[s] = ql[HILO ? s : 0] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) asm volatile("" : "+a"(qf[s]));
        if constexpr (HILO) {
#pragma unroll
            for (int s = 0; s < 16; ++s) asm volatile("" : "+a"(ql[s]));
        }
    } else {
        // workgroup-uniform resources (a per-lane base would make the compiler loop over
        // lanes); the row of this lane's column is in the offset
        const rsrc_t rq = make_rsrc(a.q, (uint32_t)a.S * a.n_q_heads * HD * 4);
        const rsrc_t rgn = make_rsrc(a.q_gain, a.q_gain ? HD * 4 : 0);
        const rsrc_t rc = make_rsrc(a.rcos, a.rcos ? (uint32_t)a.S * HD * 2 : 0);
        const rsrc_t rs = make_rsrc(a.rsin, a.rsin ? (uint32_t)a.S * HD * 2 : 0);
        const int qo = (s_idx * a.n_q_heads + kh * G + hh) * HD * 4, co = s_idx * HD * 2;
        // The operands every column shares -- the gain, and the RoPE rows of the block's
        // BQ positions when they fit (G >= 4) -- are DMA'd once into LDS stage 1, which the
        // second K/V tile takes over after the loop's first barrier; each lane then reads
        // its slices from LDS. Fetched per lane from memory they would cost 64 KiB of load
        // traffic and 256 registers per wave. Layout: [gain 1 KiB][cos BQ x 512 B][sin ...].
        constexpr bool ROPE_LDS = BQ <= 32;
        char* shr = lds + ((t0 + 1) & 1) * 2 * TILEB;
        if (wave == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rgn, (__attribute__((address_space(3))) void*)shr, 16, 16 * lane, 0, 0, 0);
        if constexpr (ROPE_LDS) {
            // BQ rows of 512 B per table from token row qb * BQ: 1 KiB per wave instruction,
            // the 16-byte chunk c of row r at c ^ (r % 8), so the rows a quarter-wave reads
            // (up to 4 positions, 512 B apart) fall on distinct banks
            constexpr int PER_WAVE = (BQ / 2 + 3) / 4;
#pragma unroll
            for (int j = 0; j < PER_WAVE; ++j) {
                const int ins = 4 * j + wave;  // the table's ins-th KiB
                if (ins < BQ / 2) {
                    const int rr = 2 * ins + (lane >> 5);
                    const int go = (qb * BQ * 512) + 512 * rr + 16 * ((lane & 31) ^ (rr & 7));
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        rc, (__attribute__((address_space(3))) void*)(shr + 1024 + 1024 * ins), 16, go, 0, 0, 0);
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(
                        rs, (__attribute__((address_space(3))) void*)(shr + 1024 + BQ * 512 + 1024 * ins), 16, go, 0, 0, 0);
                }
            }
        }
        // every remaining operand load first (one memory round trip), then the arithmetic
        float x[16][8];
        float8v cv[8], sv[8];
#pragma unroll
        for (int s = 0; s < 16; ++s) {
            const float8v v = bload_f8(rq, qo + (16 * s + 8 * h) * 4);
#pragma unroll
            for (int i = 0; i < 8; ++i) x[s][i] = v[i];
        }
        if constexpr (!ROPE_LDS) {
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                cv[s] = bload_f8(rc, co + (16 * s + 8 * h) * 4);
                sv[s] = bload_f8(rs, co + (16 * s + 8 * h) * 4);
            }
        }
        // the first K/V tile is issued behind the q operands (loads complete in order), so
        // it lands while q is prepared without delaying the q data
        if (t0 < t1) issue(t0, t0 & 1);
        if (KLO && t0 < t1) issue_klo(t0);
        // all but tile t0's 16 (+ 8 K low)
        if (t0 >= t1) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        else if constexpr (KLO) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        __syncthreads();  // every wave's share of the LDS operands
        const float* gl = reinterpret_cast<const float*>(shr) + 8 * h;
        auto gain8 = [&](int s) {
            const float4v g0 = *reinterpret_cast<const float4v*>(gl + 16 * s);
            const float4v g1 = *reinterpret_cast<const float4v*>(gl + 16 * s + 4);
            return float8v{g0[0], g0[1], g0[2], g0[3], g1[0], g1[1], g1[2], g1[3]};
        };
        if constexpr (ROPE_LDS) {
            const char* cl = shr + 1024 + pl * 512;
            const char* sl = cl + BQ * 512;
            const int sw = pl & 7;
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const int c0i = 16 * ((4 * s + 2 * h) ^ sw), c1i = 16 * ((4 * s + 2 * h + 1) ^ sw);
                const float4v c0 = *reinterpret_cast<const float4v*>(cl + c0i);
                const float4v c1 = *reinterpret_cast<const float4v*>(cl + c1i);
                const float4v s0 = *reinterpret_cast<const float4v*>(sl + c0i);
                const float4v s1 = *reinterpret_cast<const float4v*>(sl + c1i);
                cv[s] = float8v{c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
                sv[s] = float8v{s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
            }
        }
        if (!a.rcos) {
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                cv[s] = float8v{1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
                sv[s] = float8v{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            }
        }
        if (a.q_gain) {
            float se = 0.0f, so = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; ++s)
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    se = __builtin_fmaf(x[2 * s][i], x[2 * s][i], se);
                    so = __builtin_fmaf(x[2 * s + 1][i], x[2 * s + 1][i], so);
                }
            const float ss = add32(se) + add32(so);
            const float rsq = 1.0f / sqrtf(ss / (float)HD + a.eps);  // x * rs * w, as the reference kernels
#pragma unroll
            for (int s = 0; s < 16; ++s) {
                const float8v gv = gain8(s);
#pragma unroll
                for (int i = 0; i < 8; ++i) x[s][i] = x[s][i] * rsq * gv[i];
            }
        }
#pragma unroll
        for (int s = 0; s < 8; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float x0 = x[s][i], x1 = x[s + 8][i];
                x[s][i] = pin(__builtin_fmaf(x0, cv[s][i], -(x1 * sv[s][i])));
                x[s + 8][i] = pin(__builtin_fmaf(x1, cv[s][i], x0 * sv[s][i]));
            }
#pragma unroll
        for (int s = 0; s < 16; ++s)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                qf[s][i] = col_ok ? (half_t)x[s][i] : (half_t)0.0f;
                if constexpr (HILO) ql[s][i] = col_ok ? (half_t)(x[s][i] - (float)qf[s][i]) : (half_t)0.0f;
            }
        // q is only ever an MFMA B operand, which may sit in AGPRs: that leaves the VGPRs to
        // the O^T accumulators, the scores and the LDS operand batches
#pragma unroll
        for (int s = 0; s < 16; ++s) asm volatile("" : "+a"(qf[s]));
        if constexpr (HILO) {
#pragma unroll
            for (int s = 0; s < 16; ++s) asm volatile("" : "+a"(ql[s]));
        }
    }

    // ---- key ranges: this wave [w_lo, wp1], this column [col_lo, pos]
    const int wp0 = p0 + (32 * wave) / G;
    const int wp1 = min(p0 + (32 * wave + 31) / G, T_total - 1);
    const int w_lo = a.window > 0 ? max(0, wp0 + 1 - a.window) : 0;
    const int col_lo = a.window > 0 ? pos + 1 - a.window : 0;

    float16v oacc[8];  // O^T[32dt + 8(r/4) + 4h + r%4][column]
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[dt] = float16v{};
    float m_use = kNegInf, l_run = 0.0f;
    bool started = false;

    // transposed V reads: 16-lane group (h, half16), lane m supplies row 4h + m/4 (+8, +16u),
    // dims 32dt + 16 half16 + 4(m%4) .. +3
    const int m16 = lane & 15, half16 = (lane >> 4) & 1;
    const int vr0 = 4 * h + (m16 >> 2);
    const int vc0 = 2 * half16 + ((m16 & 3) >> 1);  // chunk within a 32-dim tile
    const int vb0 = 8 * (m16 & 1);                   // byte within the chunk
    const int vsw = vswz(vr0);                        // rows 16u + vr0 (+8) share r % 4

    for (int t = t0; t < t1; ++t) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's part of tile t is in LDS
        __syncthreads();                                    // all parts; tile t-1 fully consumed
        if (t + 1 < t1) issue(t + 1, (t + 1) & 1);
        const int kb = wg_lo + t * KT;
        const bool live = !(kb > wp1 || kb + KT - 1 < w_lo);  // a key of this tile for this wave
        if constexpr (!KLO) {
            if (!live) continue;
        }
        const char* K = lds + (t & 1) * 2 * TILEB;
        const char* V = K + TILEB;

        // S^T = K . Q^T: two 32-key sub-tiles, 16 k-steps of 16 dims. The two accumulator
        // chains alternate (a chain of dependent MFMAs issues at half rate), and the A
        // operands are read in batches ahead of their MFMAs. With KLO each K operand is the
        // f16 pair (high, low) of an f32 cache row, and q . k = q . k_hi + q . k_lo to f32
        // accuracy: one more MFMA per operand.
        float16v sacc[2] = {float16v{}, float16v{}};
        if (live) {
            const char* krow0 = K + n32 * ROWB;
            const char* krow1 = K + (32 + n32) * ROWB;
            const char* klrow0 = lds + 4 * TILEB + n32 * ROWB;
            const char* klrow1 = klrow0 + 32 * ROWB;
#pragma unroll
            for (int s0 = 0; s0 < 16; s0 += NB) {
                half8 kv0[NB], kv1[NB], kl0[KLO ? NB : 1], kl1[KLO ? NB : 1];
#pragma unroll
                for (int s = 0; s < NB; ++s) {
                    const int cb = 16 * ((2 * (s0 + s) + h) ^ n32);
                    kv0[s] = *reinterpret_cast<const half8*>(krow0 + cb);
                    kv1[s] = *reinterpret_cast<const half8*>(krow1 + cb);
                    if constexpr (KLO) {
                        kl0[s] = *reinterpret_cast<const half8*>(klrow0 + cb);
                        kl1[s] = *reinterpret_cast<const half8*>(klrow1 + cb);
                    }
                }
#pragma unroll
                for (int s = 0; s < NB; ++s) {
                    sacc[0] = mfma32(kv0[s], qf[s0 + s], sacc[0]);
                    if constexpr (HILO) sacc[0] = mfma32(kv0[s], ql[s0 + s], sacc[0]);
                    sacc[1] = mfma32(kv1[s], qf[s0 + s], sacc[1]);
                    if constexpr (HILO) sacc[1] = mfma32(kv1[s], ql[s0 + s], sacc[1]);
                    if constexpr (KLO) {
                        sacc[0] = mfma32(kl0[s], qf[s0 + s], sacc[0]);
                        sacc[1] = mfma32(kl1[s], qf[s0 + s], sacc[1]);
                    }
                }
            }
            // keep AHEAD LDS reads ahead of the score MFMAs (masks: 0x100 DS read, 0x008 MFMA)
            __builtin_amdgcn_sched_group_barrier(0x100, RPU * AHEAD, 0);
#pragma unroll
            for (int i = 0; i < 32 - AHEAD; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, MPU, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, RPU, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, MPU * AHEAD, 0);
        }
        if constexpr (KLO) {
            __syncthreads();  // every wave has its scores: the K low stage takes tile t + 1
            if (t + 1 < t1) issue_klo(t + 1);
            if (!live) continue;
        }

        // scores of this lane: key kb + 4h + 32kt + 8(r/4) + r%4 of its column, log2 domain;
        // tiles inside every column's range skip the per-element mask
        const bool masked = (kb + KT - 1 > wp0) || (a.window > 0 && kb < wp1 + 1 - a.window);
        if (masked) {
            const int rel_hi = pos - (kb + 4 * h), rel_lo = col_lo - (kb + 4 * h);
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int o = 32 * kt + 8 * (r >> 2) + (r & 3);
                    sacc[kt][r] = (o <= rel_hi && o >= rel_lo) ? sacc[kt][r] : kNegInf;
                }
        }
        float mloc = kNegInf;  // max of the raw scores, scaled once (scale > 0)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, sacc[kt][r]);
        mloc = max32(mloc) * a.scale_log2;  // the column's other half sits in lane ^ 32
        // move the running maxima only when a score passes one by more than 2^kMaxLag
        const bool bump = mloc > m_use + kMaxLag;
        if (__any(bump)) {
            const float m_new = fmaxf(m_use, mloc);
            const float corr = m_use == kNegInf ? 0.0f : fexp2(m_use - m_new);
            l_run *= corr;
            if (started) {
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) oacc[dt] *= corr;
            }
            m_use = m_new;
        }
        started = true;
        const float msub = m_use == kNegInf ? 0.0f : m_use;
        half8 pb[4];
        float ps = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float pv = fexp2(__builtin_fmaf(sacc[u >> 1][8 * (u & 1) + i], a.scale_log2, -msub));
                ps += pv;
                pb[u][i] = (half_t)pv;
            }
        l_run += ps;

        // O^T += V^T . P^T over four 16-key steps; k-slot i < 4 is key 16u + 4h + i,
        // i >= 4 is key 16u + 8 + 4h + i - 4, matching the S^T accumulator rows in pb
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int ra = 16 * u + vr0, rb = ra + 8;
            half8 av[8];
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                const int ch = 4 * dt + vc0;
                const half4 lo = lds_tr16(reinterpret_cast<const half_t*>(V + ra * ROWB + 16 * (ch ^ vsw) + vb0));
                const half4 hi = lds_tr16(reinterpret_cast<const half_t*>(V + rb * ROWB + 16 * (ch ^ vsw) + vb0));
                av[dt] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            }
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) oacc[dt] = mfma32(av[dt], pb[u], oacc[dt]);
        }
        // transposed V reads kept kPvAhead MFMAs ahead of the P.V MFMAs, two reads per MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * kPvAhead, 0);
#pragma unroll
        for (int i = 0; i < 32 - kPvAhead; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kPvAhead, 0);
    }

    // ---- epilogue: column sum over both halves, normalise, srq, store 4 dims at a time
    const float l_tot = add32(l_run);
    if (SPLITK && n_pieces > 1) {  // a piece of a split query block: O / l in f16 and (m, l) in f32
        const size_t blk = ((size_t)kh * a.n_qblocks + qb) * a.max_pieces + piece;
        const float inv_p = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        // one 1 KiB run per store instruction: [wave][dt][j pair][lane] half8
        half_t* po = a.part_o + blk * (NCOL * HD) + (size_t)wave * (32 * HD) + 8 * lane;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int jp = 0; jp < 2; ++jp) store_part8<true>(po + (2 * dt + jp) * 512, oacc[dt], 8 * jp, inv_p);
        if (h == 0) a.part_ml[blk * NCOL + c] = make_float2(m_use, l_tot);
        return;
    }
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if constexpr (sizeof(OUTT) == 2) {
        // f16 rows through LDS: each wave stages its 32 output rows (528-byte stride: the
        // 8-byte writes of a store instruction fall on distinct banks), then stores two whole
        // 512-byte rows an instruction. Written straight from the accumulator layout, every
        // store instruction put 16 bytes into each of 32 rows.
        constexpr int OSTR = HD * 2 + 16;
        __syncthreads();  // every wave is done with the last tile's K/V
        char* ost = lds + wave * 32 * OSTR;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4v v = float4v{oacc[dt][4 * j], oacc[dt][4 * j + 1], oacc[dt][4 * j + 2],
                                          oacc[dt][4 * j + 3]} * inv;
                store4(reinterpret_cast<half_t*>(ost + n32 * OSTR) + 32 * dt + 8 * j + 4 * h, srq4(v, a.out_q));
            }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int rr = 2 * i + h, cc = 32 * wave + rr;  // lanes 32h..: the wave's row rr
            const int so = qb * BQ + cc / G;
            const half8 val = *reinterpret_cast<const half8*>(ost + rr * OSTR + 16 * n32);
            if (so < a.S)
                *reinterpret_cast<half8*>(reinterpret_cast<half_t*>(a.out) +
                                          ((size_t)so * a.n_q_heads + kh * G + cc % G) * HD + 8 * n32) = val;
        }
    } else if (col_ok) {
        OUTT* orow = reinterpret_cast<OUTT*>(a.out) + ((size_t)s_idx * a.n_q_heads + kh * G + hh) * HD;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4v v = float4v{oacc[dt][4 * j], oacc[dt][4 * j + 1], oacc[dt][4 * j + 2],
                                          oacc[dt][4 * j + 3]} * inv;
                store4(orow + 32 * dt + 8 * j + 4 * h, srq4(v, a.out_q));
            }
    }
}

// ---------------------------------------------------------------- hd 512
// prefill_kernel_w32d: hd 512 (the global layers of Gemma 4 E2B) on the 32-column scheme.
// 32 columns x 512 dims would take 256 accumulator and 128 q registers a wave, so the dims
// are split over a pair of waves: wave d of pair p holds the 32 columns 32p .. 32p + 31 (64
// per workgroup: G heads x 64/G positions) over dims 256d .. 256d + 255. Each wave forms the
// partial scores of its dims (S_d^T = K_d . Q_d^T, 16 MFMAs a 32-key tile), the pair adds
// them through LDS (both waves then hold S_0 + S_1 and run the same softmax), and each wave
// accumulates O^T for its own dims -- per wave the registers and the LDS bytes per MFMA of
// the hd-256 kernel. Tiles of 32 keys (1 KiB rows: K and V 32 KiB each, double buffered:
// 128 KiB of LDS, plus 16 KiB for the score exchange) are DMA'd as in prefill_kernel_w32.
// q comes prepared in f16 (qprep_row512_kernel; the RoPE pairs (i, i + 256) would span both waves).
template <int G, typename OUTT, bool HILO, bool KLO>
__global__ __launch_bounds__(256) void prefill_kernel_w32d(PrefillArgs a) {
    constexpr int HD = 512, KT = 32, NCOL = 64, BQ = NCOL / G;
    constexpr int QMF = HILO ? 2 : 1;
    constexpr int MPU = QMF + (KLO ? 1 : 0);  // score MFMAs per K operand (pair)
    constexpr int ROWB = HD * 2;      // 1 KiB rows
    constexpr int TILEB = KT * ROWB;  // one K or V tile: 32 KiB
    // [buffer][K, V], then the score exchange (16 KiB); with KLO that last region is a whole
    // tile and holds the K low parts of the current tile until every wave has formed its
    // scores, then the exchange, then the next tile's K low parts (160 KiB in all)
    __shared__ __attribute__((aligned(1024))) char lds[2 * 2 * TILEB + (KLO ? TILEB : 4 * 4096)];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pr = wave >> 1, dh = wave & 1;  // pair (columns), dim half
    const int n32 = lane & 31, h = lane >> 5;
    const int T_total = a.start_pos + a.S;
    const PrefillUnit wu = prefill_unit<BQ, KT>(a, lane);
    const int kh = wu.kh, qb = wu.qb, piece = wu.piece, n_pieces = wu.n_pieces;

    const int p0 = a.start_pos + qb * BQ;
    const int kv_hi = min(p0 + BQ, T_total);
    const int wg_lo = a.window > 0 ? max(0, p0 + 1 - a.window) : 0;
    const int n_tiles = (kv_hi - wg_lo + KT - 1) / KT;
    int t0 = 0, t1 = n_tiles;
    if (a.split_tiles > 0) {
        t0 = piece * a.split_tiles;
        t1 = min(t0 + a.split_tiles, n_tiles);
    }

    // ---- this lane's query column (head hh, position offset pl) and 8-dim half h
    const int c = 32 * pr + n32;
    const int hh = c % G, pl = c / G;
    const int s_raw = qb * BQ + pl;
    const bool col_ok = s_raw < a.S;
    const int s_idx = col_ok ? s_raw : a.S - 1;
    const int pos = a.start_pos + s_idx;

    // K/V rows through buffer resources (rows >= kv_hi read as zeros); row r of a tile holds
    // chunk x at place x ^ (r % 32) (K) or x ^ vswz(r) (V): wave w moves rows 8w .. 8w + 7
    const int rowg = a.n_kv_heads * HD * 2;
    const rsrc_t rk = make_rsrc(reinterpret_cast<const half_t*>(a.kc) + (size_t)kh * HD, (uint32_t)(kv_hi - a.kv_row0) * rowg);
    const rsrc_t rv = make_rsrc(reinterpret_cast<const half_t*>(a.vc) + (size_t)kh * HD, (uint32_t)(kv_hi - a.kv_row0) * rowg);
    auto issue = [&](int t, int buf) {
        const int kb = wg_lo + t * KT - a.kv_row0;
        char* kdst = lds + buf * 2 * TILEB;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = 8 * wave + j;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(kdst + r * ROWB), 16,
                                                     (kb + r) * rowg + 16 * (lane ^ (r & 31)), 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(kdst + TILEB + r * ROWB),
                                                     16, (kb + r) * rowg + 16 * (lane ^ vswz(r)), 0, 0, 0);
        }
    };
    const rsrc_t rkl = make_rsrc(KLO ? reinterpret_cast<const half_t*>(a.kclo) + (size_t)kh * HD : nullptr,
                                 KLO ? (uint32_t)(kv_hi - a.kv_row0) * rowg : 0u);
    auto issue_klo = [&](int t) {
        const int kb = wg_lo + t * KT - a.kv_row0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = 8 * wave + j;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rkl, (__attribute__((address_space(3))) void*)(lds + 4 * TILEB + r * ROWB), 16,
                                                     (kb + r) * rowg + 16 * (lane ^ (r & 31)), 0, 0, 0);
        }
    };

    // ---- q: lane (column c, half h) holds dims 256 dh + 16s + 8h .. +7 (s < 16), the B
    // operand layout; the loads go out before the first tile's
    half8 qf[16], ql[HILO ? 16 : 1];
    {
        const rsrc_t rq = make_rsrc(a.q16, (uint32_t)a.S * a.n_q_heads * HD * 2);
        const int qo = (s_idx * a.n_q_heads + kh * G + hh) * ROWB + 512 * dh + 16 * h;
#pragma unroll
        for (int s = 0; s < 16; ++s) qf[s] = bload_h8(rq, qo + 32 * s);
        if constexpr (HILO) {
            const rsrc_t rql = make_rsrc(a.q16lo, (uint32_t)a.S * a.n_q_heads * HD * 2);
#pragma unroll
            for (int s = 0; s < 16; ++s) ql[s] = bload_h8(rql, qo + 32 * s);
        }
        if (t0 < t1) issue(t0, t0 & 1);
        if (KLO && t0 < t1) issue_klo(t0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (!col_ok) {
#pragma unroll
            for (int s = 0; s < 16; ++s) qf[s] = ql[HILO ? s : 0] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
#pragma unroll
        for (int s = 0; s < 16; ++s) asm volatile("" : "+a"(qf[s]));
        if constexpr (HILO) {
#pragma unroll
            for (int s = 0; s < 16; ++s) asm volatile("" : "+a"(ql[s]));
        }
    }

    // ---- key ranges: this pair [w_lo, wp1], this column [col_lo, pos]
    const int wp0 = p0 + (32 * pr) / G;
    const int wp1 = min(p0 + (32 * pr + 31) / G, T_total - 1);
    const int w_lo = a.window > 0 ? max(0, wp0 + 1 - a.window) : 0;
    const int col_lo = a.window > 0 ? pos + 1 - a.window : 0;

    // transposed V reads, as prefill_kernel_w32's, in this wave's dim half
    const int m16 = lane & 15, half16 = (lane >> 4) & 1;
    const int vr0 = 4 * h + (m16 >> 2);
    const int vc0 = 2 * half16 + ((m16 & 3) >> 1);
    const int vb0 = 8 * (m16 & 1);
    const int vsw = vswz(vr0);
    float* xme = reinterpret_cast<float*>(lds + 4 * TILEB) + wave * 1024;  // [r/4][lane][4]
    const float* xother = reinterpret_cast<const float*>(lds + 4 * TILEB) + (wave ^ 1) * 1024;

    float16v oacc[8];  // O^T[256 dh + 32dt + 8(r/4) + 4h + r%4][column]
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[dt] = float16v{};
    float m_use = kNegInf, l_run = 0.0f;
    bool started = false;
    for (int t = t0; t < t1; ++t) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's rows of tile t are in LDS
        __syncthreads();                                    // all rows; tile t-1 and the exchange consumed
        if (t + 1 < t1) issue(t + 1, (t + 1) & 1);
        const int kb = wg_lo + t * KT;
        const bool live = !(kb > wp1 || kb + KT - 1 < w_lo);  // pair-uniform: a key of the tile for the pair
        const char* K = lds + (t & 1) * 2 * TILEB;
        const char* V = K + TILEB;
        float16v sacc = float16v{};
        if (live) {
            // S_dh^T = K_dh . Q_dh^T over 16 k-steps of 16 dims (with KLO, K high then low parts)
            const char* krow = K + n32 * ROWB;
            const char* klrow = lds + 4 * TILEB + n32 * ROWB;
#pragma unroll
            for (int s0 = 0; s0 < 16; s0 += 4) {
                half8 kv[4], kl[KLO ? 4 : 1];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int cb = 16 * ((32 * dh + 2 * (s0 + s) + h) ^ n32);
                    kv[s] = *reinterpret_cast<const half8*>(krow + cb);
                    if constexpr (KLO) kl[s] = *reinterpret_cast<const half8*>(klrow + cb);
                }
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    sacc = mfma32(kv[s], qf[s0 + s], sacc);
                    if constexpr (HILO) sacc = mfma32(kv[s], ql[s0 + s], sacc);
                    if constexpr (KLO) sacc = mfma32(kl[s], qf[s0 + s], sacc);
                }
            }
            if constexpr (!KLO) {
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
                for (int i = 0; i < 14; ++i) {
                    __builtin_amdgcn_sched_group_barrier(0x008, MPU, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 2 * MPU, 0);
            }
        }
        if constexpr (KLO) __syncthreads();  // K low parts consumed: the exchange may overwrite them
        if (live) {
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4)
                *reinterpret_cast<float4v*>(xme + (r4 * 64 + lane) * 4) =
                    float4v{sacc[4 * r4], sacc[4 * r4 + 1], sacc[4 * r4 + 2], sacc[4 * r4 + 3]};
        }
        __syncthreads();  // the partner's partial scores
        if (live) {
            // S = S_0 + S_1 in both waves of the pair (the same sums in the same order)
#pragma unroll
            for (int r4 = 0; r4 < 4; ++r4) {
                const float4v o = *reinterpret_cast<const float4v*>(xother + (r4 * 64 + lane) * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) sacc[4 * r4 + i] = dh == 0 ? sacc[4 * r4 + i] + o[i] : o[i] + sacc[4 * r4 + i];
            }
        }
        if constexpr (KLO) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __syncthreads();  // every exchange read done: the region takes tile t + 1's K low parts
            if (t + 1 < t1) issue_klo(t + 1);
        }
        if (!live) continue;
        // scores of this lane: key kb + 4h + 8(r/4) + r%4 of its column, log2 domain
        const bool masked = (kb + KT - 1 > wp0) || (a.window > 0 && kb < wp1 + 1 - a.window);
        if (masked) {
            const int rel_hi = pos - (kb + 4 * h), rel_lo = col_lo - (kb + 4 * h);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int o = 8 * (r >> 2) + (r & 3);
                sacc[r] = (o <= rel_hi && o >= rel_lo) ? sacc[r] : kNegInf;
            }
        }
        float mloc = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, sacc[r]);
        mloc = max32(mloc) * a.scale_log2;
        const bool bump = mloc > m_use + kMaxLag;  // the running maxima move only past 2^kMaxLag
        if (__any(bump)) {
            const float m_new = fmaxf(m_use, mloc);
            const float corr = m_use == kNegInf ? 0.0f : fexp2(m_use - m_new);
            l_run *= corr;
            if (started) {
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) oacc[dt] *= corr;
            }
            m_use = m_new;
        }
        started = true;
        const float msub = m_use == kNegInf ? 0.0f : m_use;
        half8 pb[2];
        float ps = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float pv = fexp2(__builtin_fmaf(sacc[8 * u + i], a.scale_log2, -msub));
                ps += pv;
                pb[u][i] = (half_t)pv;
            }
        l_run += ps;

        // O^T_dh += V_dh^T . P^T over two 16-key steps
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int ra = 16 * u + vr0, rb = ra + 8;
#pragma unroll
            for (int d0 = 0; d0 < 8; d0 += 4) {
                half8 av[4];
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) {
                    const int ch = 32 * dh + 4 * (d0 + dd) + vc0;
                    const half4 lo = lds_tr16(reinterpret_cast<const half_t*>(V + ra * ROWB + 16 * (ch ^ vsw) + vb0));
                    const half4 hi = lds_tr16(reinterpret_cast<const half_t*>(V + rb * ROWB + 16 * (ch ^ vsw) + vb0));
                    av[dd] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) oacc[d0 + dd] = mfma32(av[dd], pb[u], oacc[d0 + dd]);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 14; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }

    // ---- epilogue: this wave's 256 dims of its 32 columns
    const float l_tot = add32(l_run);
    if (n_pieces > 1) {  // a piece of a split query block: O / l in f16, (m, l) from wave dh 0
        const size_t blk = ((size_t)kh * a.n_qblocks + qb) * a.max_pieces + piece;
        const float inv_p = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        half_t* po = a.part_o + blk * (NCOL * HD) + (size_t)wave * (32 * 256) + 8 * lane;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int jp = 0; jp < 2; ++jp) store_part8<false>(po + (2 * dt + jp) * 512, oacc[dt], 8 * jp, inv_p);
        if (h == 0 && dh == 0) a.part_ml[blk * NCOL + c] = make_float2(m_use, l_tot);
        return;
    }
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if constexpr (sizeof(OUTT) == 2) {
        // f16 rows through LDS, as prefill_kernel_w32 stores them: each wave stages the 256
        // dims of its 32 columns (528-byte stride), then stores two 512-byte runs an instruction
        constexpr int OSTR = 256 * 2 + 16;
        __syncthreads();  // every wave is done with the last tile's K/V
        char* ost = lds + wave * 32 * OSTR;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4v v = float4v{oacc[dt][4 * j], oacc[dt][4 * j + 1], oacc[dt][4 * j + 2],
                                          oacc[dt][4 * j + 3]} * inv;
                store4(reinterpret_cast<half_t*>(ost + n32 * OSTR) + 32 * dt + 8 * j + 4 * h, srq4(v, a.out_q));
            }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int rr = 2 * i + h, cc = 32 * pr + rr;  // lanes 32h..: the wave's row rr
            const int so = qb * BQ + cc / G;
            const half8 val = *reinterpret_cast<const half8*>(ost + rr * OSTR + 16 * n32);
            if (so < a.S)
                *reinterpret_cast<half8*>(reinterpret_cast<half_t*>(a.out) +
                                          ((size_t)so * a.n_q_heads + kh * G + cc % G) * HD + 256 * dh + 8 * n32) = val;
        }
    } else if (col_ok) {
        OUTT* orow = reinterpret_cast<OUTT*>(a.out) + ((size_t)s_idx * a.n_q_heads + kh * G + hh) * HD + 256 * dh;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4v v = float4v{oacc[dt][4 * j], oacc[dt][4 * j + 1], oacc[dt][4 * j + 2],
                                          oacc[dt][4 * j + 3]} * inv;
                store4(orow + 32 * dt + 8 * j + 4 * h, srq4(v, a.out_q));
            }
    }
}

// prefill_kernel_w32h: hd 512 with every wave holding all 512 dims of its 32 columns (128
// columns a workgroup: G heads x 128/G positions), the GEMM form's plain mode (f16 q from
// qprep_row512_kernel, f16 caches). Per 32-key tile a wave runs 32 score MFMAs (two accumulator
// chains over alternate k-steps, added at the end) and 32 P.V MFMAs into 16 O^T tiles of
// 32 dims -- 256 accumulator registers, which live in AGPRs, with q (128 registers) in
// VGPRs: one wave a SIMD, no partner wave and no per-tile score exchange, and each K/V
// tile staged in LDS serves twice the columns of prefill_kernel_w32d's. The tile's LDS
// layout, DMA, masks and softmax are prefill_kernel_w32d's.
// acc += a . b with the accumulator in AGPRs (the file's MFMAs are built in VGPR form). The
// leading s_nop covers a VALU write of a or b just before (2 wait states); the MFMA pipe
// takes 32 cycles an instruction, so it costs no issue slot the pipe could have used.
__device__ __forceinline__ void mfma32_acc(float16v& acc, half8 a, half8 b) {
    asm("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

template <int G, typename OUTT, bool QSTAGE, bool OSTAGE>
__global__ __launch_bounds__(256) void prefill_kernel_w32h(PrefillArgs a) {
    constexpr int HD = 512, KT = 32, NCOL = 128, BQ = NCOL / G;
    constexpr int ROWB = HD * 2;      // 1 KiB rows
    constexpr int TILEB = KT * ROWB;  // one K or V tile: 32 KiB
    constexpr int OSTR = HD * 2 + 16;  // the epilogue's staged f16 output rows (1040 B apart)
    constexpr int LDS_BYTES = !OSTAGE || 2 * 2 * TILEB > 4 * 32 * OSTR ? 2 * 2 * TILEB : 4 * 32 * OSTR;
    __shared__ __attribute__((aligned(1024))) char lds[LDS_BYTES];  // [buffer][K, V]; output rows

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n32 = lane & 31, h = lane >> 5;
    const int T_total = a.start_pos + a.S;
    const PrefillUnit wu = prefill_unit<BQ, KT>(a, lane);
    const int kh = wu.kh, qb = wu.qb, piece = wu.piece, n_pieces = wu.n_pieces;

    const int p0 = a.start_pos + qb * BQ;
    const int kv_hi = min(p0 + BQ, T_total);
    const int wg_lo = a.window > 0 ? max(0, p0 + 1 - a.window) : 0;
    const int n_tiles = (kv_hi - wg_lo + KT - 1) / KT;
    int t0 = 0, t1 = n_tiles;
    if (a.split_tiles > 0) {
        t0 = piece * a.split_tiles;
        t1 = min(t0 + a.split_tiles, n_tiles);
    }

    // ---- this lane's query column (head hh, position offset pl) and 8-dim half h
    const int c = 32 * wave + n32;
    const int hh = c % G, pl = c / G;
    const int s_raw = qb * BQ + pl;
    const bool col_ok = s_raw < a.S;
    const int s_idx = col_ok ? s_raw : a.S - 1;
    const int pos = a.start_pos + s_idx;

    // K/V rows through buffer resources (rows >= kv_hi read as zeros); wave w moves rows
    // 8w .. 8w + 7 of each, one 1 KiB row per instruction
    const int rowg = a.n_kv_heads * HD * 2;
    const rsrc_t rk = make_rsrc(reinterpret_cast<const half_t*>(a.kc) + (size_t)kh * HD, (uint32_t)(kv_hi - a.kv_row0) * rowg);
    const rsrc_t rv = make_rsrc(reinterpret_cast<const half_t*>(a.vc) + (size_t)kh * HD, (uint32_t)(kv_hi - a.kv_row0) * rowg);
    // (the lane index passes through an empty asm each time, so the 16 source offsets are
    // formed per tile rather than held in registers across the loop)
    auto issue = [&](int t, int buf) {
        const int kb = wg_lo + t * KT - a.kv_row0;
        char* kdst = lds + buf * 2 * TILEB;
        int ln = lane;
        asm volatile("" : "+v"(ln));
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int r = 8 * wave + j;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(kdst + r * ROWB), 16,
                                                     (kb + r) * rowg + 16 * (ln ^ (r & 31)), 0, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (__attribute__((address_space(3))) void*)(kdst + TILEB + r * ROWB),
                                                     16, (kb + r) * rowg + 16 * (ln ^ vswz(r)), 0, 0, 0);
        }
    };

    // ---- q: lane (column c, half h) holds dims 16s + 8h .. +7 (s < 32), the B operand
    // layout. QSTAGE (the launches with a key split, whose many pieces start at once): wave w
    // DMAs the f16 q rows of its 32 columns, whole 1 KiB rows (chunk n of a row from logical
    // chunk n ^ (column % 32)), into its 16 KiB of the LDS stage that tile t0 + 1 takes over
    // later, in two rounds of 16 rows (the stage holds half of the workgroup's 128 KiB of q),
    // and reads each round back in the B-operand layout; tile t0's DMA goes out after the
    // first round's. Loaded straight in the operand layout, every load instruction took 32
    // bytes from each of 32 rows: S 1024 global 48.2 -> 47.6 us a call with the staging.
    // Without a split the q rows load straight, all 32 loads at once behind tile t0's DMA:
    // the staged form, even compiled beside the direct one and not taken, made the S 8192
    // global kernel 684 -> 707 us (the same tile loop, instruction for instruction).
    half8 qf[32];
    {
        const rsrc_t rq = make_rsrc(a.q16, (uint32_t)a.S * a.n_q_heads * HD * 2);
        if constexpr (QSTAGE) {
            char* qs = lds + ((t0 + 1) & 1) * 2 * TILEB + wave * 16 * ROWB;
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                int ln = lane;
                asm volatile("" : "+v"(ln));
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int cj = 32 * wave + 16 * r + j;  // the column whose row this DMA moves
                    const int qo = ((qb * BQ + cj / G) * a.n_q_heads + kh * G + cj % G) * ROWB + 16 * (ln ^ (16 * r + j));
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(rq, (__attribute__((address_space(3))) void*)(qs + j * ROWB),
                                                             16, qo, 0, 0, 0);
                }
                if (r == 0 && t0 < t1) {
                    issue(t0, t0 & 1);
                    asm volatile("s_waitcnt vmcnt(16)" ::: "memory");  // the 16 q DMAs before tile t0's
                } else {
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                }
                if ((n32 >> 4) == r) {
                    const char* qrow = qs + (n32 & 15) * ROWB;
#pragma unroll
                    for (int s = 0; s < 32; ++s) qf[s] = *reinterpret_cast<const half8*>(qrow + 16 * ((2 * s + h) ^ n32));
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's 16 KiB free again
            }
        } else {
            const int qo = (s_idx * a.n_q_heads + kh * G + hh) * ROWB + 16 * h;
#pragma unroll
            for (int s = 0; s < 32; ++s) qf[s] = bload_h8(rq, qo + 32 * s);
            if (t0 < t1) issue(t0, t0 & 1);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        if (!col_ok) {
#pragma unroll
            for (int s = 0; s < 32; ++s) qf[s] = half8{0, 0, 0, 0, 0, 0, 0, 0};
        }
    }

    // ---- key ranges: this wave [w_lo, wp1], this column [col_lo, pos]
    const int wp0 = p0 + (32 * wave) / G;
    const int wp1 = min(p0 + (32 * wave + 31) / G, T_total - 1);
    const int w_lo = a.window > 0 ? max(0, wp0 + 1 - a.window) : 0;
    const int col_lo = a.window > 0 ? pos + 1 - a.window : 0;

    // LDS read offsets. K operand k-step s of this lane: row n32, chunk (2s + h) ^ n32, i.e.
    // byte kofs ^ 32s with kofs = 1024 n32 + 16 (h ^ n32). Transposed V reads (as
    // prefill_kernel_w32's): row 16u + 8i + vr0, chunk (4dt + vc0) ^ vsw, i.e. byte
    // (vofs ^ 64dt) + 1024 (16u + 8i) with vofs = 1024 vr0 + 16 (vc0 ^ vsw) + vb0. Both offsets
    // pass through an empty asm every tile, so the compiler forms the 32 + 16 XORs in the
    // loop instead of holding 48 hoisted addresses.
    const int m16 = lane & 15, half16 = (lane >> 4) & 1;
    const int vr0 = 4 * h + (m16 >> 2);
    const int vc0 = 2 * half16 + ((m16 & 3) >> 1);
    const int vb0 = 8 * (m16 & 1);
    const int kofs0 = 1024 * n32 + 16 * (h ^ n32);
    const int vofs0 = 1024 * vr0 + 16 * (vc0 ^ vswz(vr0)) + vb0;

    float16v oacc[16];  // O^T[32dt + 8(r/4) + 4h + r%4][column]
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) oacc[dt] = float16v{};
#pragma unroll
    for (int dt = 0; dt < 16; ++dt) asm volatile("" : "+a"(oacc[dt]));
    float m_use = kNegInf, l_run = 0.0f;
    bool started = false;
    for (int t = t0; t < t1; ++t) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's rows of tile t are in LDS
        __syncthreads();                                    // all rows; tile t-1 consumed
        if (t + 1 < t1) issue(t + 1, (t + 1) & 1);
        const int kb = wg_lo + t * KT;
        if (kb > wp1 || kb + KT - 1 < w_lo) continue;  // no key of this tile for this wave
        int kofs = (t & 1) * 2 * TILEB + kofs0, vofs = (t & 1) * 2 * TILEB + TILEB + vofs0;
        asm volatile("" : "+v"(kofs), "+v"(vofs));

        // S^T = K . Q^T over 32 k-steps of 16 dims, even and odd steps in two chains
        float16v se = float16v{}, so = float16v{};
        {
#pragma unroll
            for (int s0 = 0; s0 < 32; s0 += 4) {
                half8 kv[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) kv[s] = *reinterpret_cast<const half8*>(lds + (kofs ^ (32 * (s0 + s))));
#pragma unroll
                for (int s = 0; s < 4; s += 2) {
                    se = mfma32(kv[s], qf[s0 + s], se);
                    so = mfma32(kv[s + 1], qf[s0 + s + 1], so);
                }
            }
            __builtin_amdgcn_sched_group_barrier(0x100, kQkAhead, 0);
#pragma unroll
            for (int i = 0; i < 32 - kQkAhead; ++i) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x008, kQkAhead, 0);
        }
        float sacc[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[r] = se[r] + so[r];
        // scores of this lane: key kb + 4h + 8(r/4) + r%4 of its column, log2 domain
        const bool masked = (kb + KT - 1 > wp0) || (a.window > 0 && kb < wp1 + 1 - a.window);
        if (masked) {
            const int rel_hi = pos - (kb + 4 * h), rel_lo = col_lo - (kb + 4 * h);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int o = 8 * (r >> 2) + (r & 3);
                sacc[r] = (o <= rel_hi && o >= rel_lo) ? sacc[r] : kNegInf;
            }
        }
        float mloc = kNegInf;
#pragma unroll
        for (int r = 0; r < 16; ++r) mloc = fmaxf(mloc, sacc[r]);
        mloc = max32(mloc) * a.scale_log2;
        const bool bump = mloc > m_use + kMaxLag;  // the running maxima move only past 2^kMaxLag
        if (__any(bump)) {
            const float m_new = fmaxf(m_use, mloc);
            const float corr = m_use == kNegInf ? 0.0f : fexp2(m_use - m_new);
            l_run *= corr;
            if (started) {
                // one 16-register tile at a time: copied to VGPRs, scaled, pinned back into
                // AGPRs (left to itself the compiler moves all 256 through VGPRs and spills)
                asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"  // the last MFMA's writes, as in the epilogue
                             : "+a"(oacc[0]), "+a"(oacc[1]), "+a"(oacc[2]), "+a"(oacc[3]), "+a"(oacc[4]),
                               "+a"(oacc[5]), "+a"(oacc[6]), "+a"(oacc[7]), "+a"(oacc[8]), "+a"(oacc[9]),
                               "+a"(oacc[10]), "+a"(oacc[11]), "+a"(oacc[12]), "+a"(oacc[13]), "+a"(oacc[14]),
                               "+a"(oacc[15]));
#pragma unroll
                for (int dt = 0; dt < 16; ++dt) {
                    float16v x = oacc[dt];
                    asm volatile("" : "+v"(x));
                    x *= corr;
                    asm volatile("" : "+v"(x));
                    oacc[dt] = x;
                    asm volatile("" : "+a"(oacc[dt]));
                }
            }
            m_use = m_new;
        }
        started = true;
        const float msub = m_use == kNegInf ? 0.0f : m_use;
        half8 pb[2];
        float ps = 0.0f;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float pv = fexp2(__builtin_fmaf(sacc[8 * u + i], a.scale_log2, -msub));
                ps += pv;
                pb[u][i] = (half_t)pv;
            }
        l_run += ps;

        // O^T += V^T . P^T over two 16-key steps, 16 dims tiles each
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int d0 = 0; d0 < 16; d0 += 4) {
                half8 av[4];
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) {
                    const char* vp = lds + (vofs ^ (64 * (d0 + dd))) + 16 * u * ROWB;
                    const half4 lo = lds_tr16(reinterpret_cast<const half_t*>(vp));
                    const half4 hi = lds_tr16(reinterpret_cast<const half_t*>(vp + 8 * ROWB));
                    av[dd] = half8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                }
#pragma unroll
                for (int dd = 0; dd < 4; ++dd) mfma32_acc(oacc[d0 + dd], av[dd], pb[u]);
            }
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * kPvAhead, 0);
#pragma unroll
        for (int i = 0; i < 32 - kPvAhead; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, kPvAhead, 0);
    }

    // ---- epilogue: the 512 dims of this wave's 32 columns. The accumulators are read by
    // VALU instructions below, which must not issue within 18 wait states of the last MFMA
    // writing them (the compiler does not see the asm MFMAs); the asm also orders every read
    // after the wait, since each accumulator passes through it.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 3"
                 : "+a"(oacc[0]), "+a"(oacc[1]), "+a"(oacc[2]), "+a"(oacc[3]), "+a"(oacc[4]), "+a"(oacc[5]),
                   "+a"(oacc[6]), "+a"(oacc[7]), "+a"(oacc[8]), "+a"(oacc[9]), "+a"(oacc[10]), "+a"(oacc[11]),
                   "+a"(oacc[12]), "+a"(oacc[13]), "+a"(oacc[14]), "+a"(oacc[15]));
    const float l_tot = add32(l_run);
    if (n_pieces > 1) {  // a piece of a split query block: O / l in f16 and (m, l) in f32
        // blocks of 32 columns x 256 dims, [wave][dim half][dt % 8][j pair][lane] half8: the
        // layout prefill_kernel_w32d writes for its (pair, dim half) waves
        const size_t blk = ((size_t)kh * a.n_qblocks + qb) * a.max_pieces + piece;
        const float inv_p = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        half_t* po = a.part_o + blk * (NCOL * HD) + (size_t)wave * (32 * HD) + 8 * lane;
#pragma unroll
        for (int dt = 0; dt < 16; ++dt)
#pragma unroll
            for (int jp = 0; jp < 2; ++jp) store_part8<false>(po + (2 * dt + jp) * 512, oacc[dt], 8 * jp, inv_p);
        if (h == 0) a.part_ml[blk * NCOL + c] = make_float2(m_use, l_tot);
        return;
    }
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if constexpr (OSTAGE && sizeof(OUTT) == 2) {
        // f16 rows through LDS, as prefill_kernel_w32 stores them: each wave stages its 32
        // output rows, then stores one whole 1 KiB row an instruction. Launches with a key
        // split or a window take it (S 1024 global 47.0 -> 44.7 us a call, S 8192 W 512
        // 181 -> 176 us); the unsplit causal launch stores straight (with the staging its
        // S 8192 kernel took 705-709 against 684-689 us)
        __syncthreads();  // every wave is done with the last tile's K/V
        char* ost = lds + wave * 32 * OSTR;
#pragma unroll
        for (int dt = 0; dt < 16; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4v v = float4v{oacc[dt][4 * j], oacc[dt][4 * j + 1], oacc[dt][4 * j + 2],
                                          oacc[dt][4 * j + 3]} * inv;
                store4(reinterpret_cast<half_t*>(ost + n32 * OSTR) + 32 * dt + 8 * j + 4 * h, srq4(v, a.out_q));
            }
#pragma unroll
        for (int rr = 0; rr < 32; ++rr) {
            const int cc = 32 * wave + rr, so = qb * BQ + cc / G;
            const half8 val = *reinterpret_cast<const half8*>(ost + rr * OSTR + 16 * lane);
            if (so < a.S)
                *reinterpret_cast<half8*>(reinterpret_cast<half_t*>(a.out) +
                                          ((size_t)so * a.n_q_heads + kh * G + cc % G) * HD + 8 * lane) = val;
        }
    } else if (col_ok) {
        OUTT* orow = reinterpret_cast<OUTT*>(a.out) + ((size_t)s_idx * a.n_q_heads + kh * G + hh) * HD;
#pragma unroll
        for (int dt = 0; dt < 16; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4v v = float4v{oacc[dt][4 * j], oacc[dt][4 * j + 1], oacc[dt][4 * j + 2],
                                          oacc[dt][4 * j + 3]} * inv;
                store4(orow + 32 * dt + 8 * j + 4 * h, srq4(v, a.out_q));
            }
    }
}

// Merge of the pieces of split query blocks (the decode merge identity per column): with
// each piece holding o_p = O_p / l_p, out = sum_p o_p l_p 2^(m_p - M) / sum_p l_p 2^(m_p - M),
// M = max_p m_p, then srq and the output type. One workgroup per (query block, wave block of
// 32 columns x 256 dims, kv head), laid out like the partials: thread (k, lane) owns the
// lane's 8-dim runs k, k+4, .. (k < 4) of the 16 (dims tile, 4-row pair) runs, so every load
// instruction reads a contiguous 1 KiB run. At most 8 pieces. HD 256: wave block w = columns 32w..; HD 512
// (prefill_kernel_w32d, NCOL 64, and prefill_kernel_w32h, NCOL 128): columns 32(w/2)..,
// dims 256(w%2)..
template <typename OUTT, int HD, int NCOL>
__global__ __launch_bounds__(256) void prefill_merge_kernel(PrefillArgs a) {
    constexpr int KT = HD == 256 ? 64 : 32, MAXP = 8;
    const int qb = blockIdx.x, w = blockIdx.y, kh = blockIdx.z, tid = threadIdx.x;
    const int lane = tid & 63, k0 = tid >> 6;
    const int c = (HD == 256 ? 32 * w : 32 * (w >> 1)) + (lane & 31), h = lane >> 5;
    const int dbase = HD == 256 ? 0 : 256 * (w & 1);
    const int G = a.n_q_heads / a.n_kv_heads, BQ = NCOL / G;
    const int p0 = a.start_pos + qb * BQ;
    const int kv_hi = min(p0 + BQ, a.start_pos + a.S);
    const int wg_lo = a.window > 0 ? max(0, p0 + 1 - a.window) : 0;
    const int n_tiles = (kv_hi - wg_lo + KT - 1) / KT;
    const int n_pieces = max(1, (n_tiles + a.split_tiles - 1) / a.split_tiles);
    const int s_idx = qb * BQ + c / G;
    if (n_pieces <= 1) return;
    const size_t blk0 = ((size_t)kh * a.n_qblocks + qb) * a.max_pieces;
    // buffer ranges end at the block's last piece: the loads of absent pieces read zeros,
    // so all of them issue at once with no branch
    const rsrc_t rml = make_rsrc(a.part_ml + blk0 * NCOL, (uint32_t)n_pieces * NCOL * 8);
    const rsrc_t ro = make_rsrc(a.part_o + blk0 * (NCOL * HD) + (size_t)w * (32 * 256), (uint32_t)n_pieces * NCOL * HD * 2);
    float2 ml[MAXP];
    half8 ov[MAXP][4];
#pragma unroll
    for (int p = 0; p < MAXP; ++p) ml[p] = bload_f32x2(rml, (p * NCOL + c) * 8);
#pragma unroll
    for (int p = 0; p < MAXP; ++p)
#pragma unroll
        for (int i = 0; i < 4; ++i)  // run k = k0 + 4i: dims tile k/2, 4-row pair k%2
            ov[p][i] = bload_h8(ro, (p * NCOL * HD + (k0 + 4 * i) * 512 + 8 * lane) * 2);
    float wt[MAXP];
    float M = kNegInf;
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {
        if (p >= n_pieces) ml[p] = make_float2(kNegInf, 0.0f);
        M = fmaxf(M, ml[p].x);
    }
    float L = 0.0f;
#pragma unroll
    for (int p = 0; p < MAXP; ++p) {  // a piece with no attended key weighs 0
        wt[p] = ml[p].x == kNegInf ? 0.0f : ml[p].y * fexp2(ml[p].x - M);
        L += wt[p];
    }
    float4v o[8];  // o[2i + e]: rows 8e.. of run i
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = float4v{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int p = 0; p < MAXP; ++p) {
            const half8 v = ov[p][i];
            o[2 * i] += float4v{(float)v[0], (float)v[1], (float)v[2], (float)v[3]} * wt[p];
            o[2 * i + 1] += float4v{(float)v[4], (float)v[5], (float)v[6], (float)v[7]} * wt[p];
        }
    if (s_idx >= a.S) return;
    const float inv = L > 0.0f ? 1.0f / L : 0.0f;
    OUTT* orow = reinterpret_cast<OUTT*>(a.out) + ((size_t)s_idx * a.n_q_heads + kh * G + c % G) * HD + dbase;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int k = k0 + 4 * i, d = 32 * (k >> 1) + 16 * (k & 1) + 8 * e + 4 * h;
            store4(orow + d, srq4(o[2 * i + e] * inv, a.out_q));
        }
}

typedef void (*prefill_fn)(PrefillArgs);

template <int HD, int G, bool HILO, bool KLO>
static prefill_fn pick_w32_out(bool out32, bool split) {
    if constexpr (HD == 256) {
        if (split) return out32 ? prefill_kernel_w32<G, float, HILO, KLO, true> : prefill_kernel_w32<G, half_t, HILO, KLO, true>;
        return out32 ? prefill_kernel_w32<G, float, HILO, KLO, false> : prefill_kernel_w32<G, half_t, HILO, KLO, false>;
    } else {
        return out32 ? prefill_kernel_w32d<G, float, HILO, KLO> : prefill_kernel_w32d<G, half_t, HILO, KLO>;
    }
}
template <int HD, int G>
static prefill_fn pick_w32(bool out32, bool hilo, bool klo, bool split) {
    if (hilo) return klo ? pick_w32_out<HD, G, true, true>(out32, split) : pick_w32_out<HD, G, true, false>(out32, split);
    return klo ? pick_w32_out<HD, G, false, true>(out32, split) : pick_w32_out<HD, G, false, false>(out32, split);
}
template <int G>
static prefill_fn pick_w32h(bool out32, bool qstage, bool ostage) {
    if (qstage) return out32 ? prefill_kernel_w32h<G, float, true, true> : prefill_kernel_w32h<G, half_t, true, true>;
    if (ostage) return out32 ? prefill_kernel_w32h<G, float, false, true> : prefill_kernel_w32h<G, half_t, false, true>;
    return out32 ? prefill_kernel_w32h<G, float, false, false> : prefill_kernel_w32h<G, half_t, false, false>;
}
static prefill_fn pick_g_w32h(int G, bool out32, bool qstage, bool ostage) {
    switch (G) {
        case 1: return pick_w32h<1>(out32, qstage, ostage);
        case 2: return pick_w32h<2>(out32, qstage, ostage);
        case 4: return pick_w32h<4>(out32, qstage, ostage);
        case 8: return pick_w32h<8>(out32, qstage, ostage);
    }
    return nullptr;
}
template <int HD>
static prefill_fn pick_g(int G, bool out32, bool hilo, bool klo, bool split) {
    switch (G) {
        case 1: return pick_w32<HD, 1>(out32, hilo, klo, split);
        case 2: return pick_w32<HD, 2>(out32, hilo, klo, split);
        case 4: return pick_w32<HD, 4>(out32, hilo, klo, split);
        case 8: return pick_w32<HD, 8>(out32, hilo, klo, split);
    }
    return nullptr;
}

}  // namespace g4a

using namespace g4a;

// Key split for short prompts: when the query blocks alone give fewer than 2 workgroups
// per CU, long causal rows are cut into pieces of split_tiles key tiles, the longest block
// into about six pieces. Measured best piece sizes at 16 / 24 / 32 / 64 tiles in the
// longest block (S 1024, 1536, 2048, 4096 global): 3 / 3-4 / 5 / 10-13 tiles; one piece
// per CU (3 / 5 / 9 / 33) was up to 24 % slower beyond S 1024.
struct PrefillSplit {
    int split_tiles, max_pieces, n_qblocks, total_pieces;
    int kv_row0, kv_rows;  // f32 caches: the attended rows copied to f16
    // workspace layout [K16][V16][K16 low][q16][q16 low][partials][(m, l)]; base: the bytes
    // the unsplit call needs, total: with the split
    size_t kv16_bytes, q16_bytes, q16lo_bytes, o_bytes, ml_bytes, base, total;
};
// Every mode runs the 32-column kernels (hd 256: prefill_kernel_w32, hd 512:
// prefill_kernel_w32d). Some need workspace (base > 0): f32 caches the f16 (K high, V, K
// low) copy of the attended rows (kv16_kernel); hd 512 its q in f16 (qprep_row512_kernel; with
// G4A_Q_HILO the low parts too). hd 256 on f16 caches runs unsplit without a workspace
// (its q prologue fused in).
static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
// query columns a workgroup of the kernel that runs the call holds
static int prefill_ncol(int HD, bool hilo) { return HD == 256 || !hilo ? 128 : 64; }
static PrefillSplit prefill_split(const g4a_cfg* cfg, int S, int start_pos) {
    PrefillSplit p{0, 1, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    const int HD = (int)cfg->head_dim;
    if ((HD != 256 && HD != 512) || S <= 0 || cfg->n_kv_heads == 0) return p;
    const int G = (int)(cfg->n_q_heads / cfg->n_kv_heads);
    const bool hilo = (cfg->flags & G4A_Q_HILO) != 0;
    const int NCOL = prefill_ncol(HD, hilo), KT = HD == 256 ? 64 : 32;
    if (G < 1 || NCOL % G) return p;
    const int BQ = NCOL / G, kvH = (int)cfg->n_kv_heads, W = (int)cfg->window;
    if (cfg->flags & G4A_KV_F32) {
        p.kv_row0 = W > 0 && start_pos + 1 - W > 0 ? start_pos + 1 - W : 0;
        p.kv_rows = start_pos + S - p.kv_row0;
        // K high and V; K low with G4A_Q_HILO (the fused form's f32 scores)
        p.kv16_bytes = (hilo ? 3 : 2) * align256((size_t)p.kv_rows * kvH * HD * sizeof(half_t));
    }
    const size_t q16 = align256((size_t)S * cfg->n_q_heads * HD * sizeof(half_t));
    p.base = p.kv16_bytes + (HD == 512 ? q16 * (hilo ? 2 : 1) : 0);
    p.total = p.base;
    p.n_qblocks = (S + BQ - 1) / BQ;
    if ((long)p.n_qblocks * kvH >= 512) return p;
    // a sliding window bounds every block to W/KT + 1 tiles: splitting then pays its q
    // preparation and merge only while the unsplit grid leaves most CUs idle (hd 256, S 2048,
    // W 512: 34 us unsplit against 45 us split; S 1024: 32 against 27; hd 512 on
    // prefill_kernel_w32d, S 1024, W 512, 128 workgroups: 49.9 unsplit against 52.7; on
    // prefill_kernel_w32h, 64 workgroups: 76 unsplit against 43 split)
    if (W > 0 && (long)p.n_qblocks * kvH >= 128) return p;
    int max_tiles = 0;
    for (int qb = 0; qb < p.n_qblocks; ++qb) {
        const int p0 = start_pos + qb * BQ;
        const int hi = p0 + BQ < start_pos + S ? p0 + BQ : start_pos + S;
        const int lo = W > 0 && p0 + 1 - W > 0 ? p0 + 1 - W : 0;
        const int nt = (hi - lo + KT - 1) / KT;
        if (nt > max_tiles) max_tiles = nt;
    }
    int st = (max_tiles * 5 + 31) / 32;
    // at least 2 tiles a piece, 4 for prefill_kernel_w32h's 32-key tiles (hd 512, S 1024,
    // W 512, 17-tile blocks: 3 tiles a piece 53.5 us a call, 4 tiles 43.4, 5 tiles 47.4;
    // global, 32-tile blocks: 5 tiles 48.1 us, 7 tiles 52.6)
    const int st_min = HD == 512 && NCOL == 128 ? 4 : 2;
    if (st < st_min) st = st_min;
    if (st < (max_tiles + 7) / 8) st = (max_tiles + 7) / 8;  // the merge takes <= 8 pieces
    const int pieces = (max_tiles + st - 1) / st;
    if (pieces <= 1) return p;
    p.split_tiles = st;
    p.max_pieces = pieces;
    p.total_pieces = 0;
    for (int qb = 0; qb < p.n_qblocks; ++qb) {
        const int p0 = start_pos + qb * BQ;
        const int hi = p0 + BQ < start_pos + S ? p0 + BQ : start_pos + S;
        const int lo = W > 0 && p0 + 1 - W > 0 ? p0 + 1 - W : 0;
        const int nt = (hi - lo + KT - 1) / KT;
        p.total_pieces += nt > st ? (nt + st - 1) / st : 1;
    }
    const size_t slots = (size_t)kvH * p.n_qblocks * pieces * NCOL;
    p.q16_bytes = q16;
    p.q16lo_bytes = hilo ? q16 : 0;
    p.o_bytes = slots * HD * sizeof(half_t);
    p.ml_bytes = align256(slots * sizeof(float2));
    p.total = p.kv16_bytes + p.q16_bytes + p.q16lo_bytes + p.o_bytes + p.ml_bytes;
    return p;
}

namespace g4a {
// f32 caches as MFMA operands, n8 groups of 8 values: V and K as f16 (round to nearest
// even), which is the GEMM form's own conversion (srqh_b with step 0 on both caches before
// the score and P.V GEMMs, prefill_gpu.py:286-288); with klo also the low parts of K,
// k_lo = f16(k - f16(k)) -- the difference is exact in f32 and f16(k) + k_lo is k to within
// 2^-22 |k| -- so the fused form (f32 q and f32 caches, attn_prefill) forms q . k_hi + q . k_lo
// at f32 accuracy: with scale 1.0 and |q.k| in the tens, K rounded to f16 alone moves its
// scores by ~0.1. V stays f16 in both forms: its rounding (2^-11 relative) is that of P's
// f16 operand.
__global__ __launch_bounds__(256) void kv16_kernel(const float* kc, const float* vc, half_t* ko, half_t* vo,
                                                   half_t* klo, size_t n8) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n8) return;
    const float4v* k4 = reinterpret_cast<const float4v*>(kc) + 2 * i;
    const float4v* v4 = reinterpret_cast<const float4v*>(vc) + 2 * i;
    const float4v k0 = k4[0], k1 = k4[1], v0 = v4[0], v1 = v4[1];
    const float8v k = float8v{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
    half8 hi, lo;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        hi[j] = (half_t)k[j];
        lo[j] = (half_t)(k[j] - (float)hi[j]);
    }
    reinterpret_cast<half8*>(ko)[i] = hi;
    if (klo) reinterpret_cast<half8*>(klo)[i] = lo;
    reinterpret_cast<half8*>(vo)[i] = half8{(half_t)v0[0], (half_t)v0[1], (half_t)v0[2], (half_t)v0[3],
                                            (half_t)v1[0], (half_t)v1[1], (half_t)v1[2], (half_t)v1[3]};
}
}  // namespace g4a

extern "C" size_t g4a_prefill_ws_bytes(const g4a_cfg* cfg, int S, int start_pos) {
    if (!cfg) return 0;
    return prefill_split(cfg, S, start_pos).total;  // the split's when the call splits
}

extern "C" int g4a_prefill(const g4a_cfg* cfg, int S, int start_pos, const float* q,
                           const float* q_gain, const float* rope_cos, const float* rope_sin,
                           const void* k_cache, const void* v_cache, void* out, void* ws,
                           size_t ws_bytes, void* stream) {
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
    // f32 caches need their f16 (K high, V, K low) copy and hd 512 its f16 q in the
    // workspace (prefill_split's base); hd 256 on f16 caches runs without one
    const PrefillSplit sp = prefill_split(cfg, S, start_pos);
    const bool ws_ok = ws && (uintptr_t)ws % 256 == 0;
    if (sp.base > 0 && !(ws_ok && ws_bytes >= sp.base)) {
        set_error("%s needs a 256-byte aligned workspace of at least %zu bytes (g4a_prefill_ws_bytes), got %zu",
                  kv32 ? "a prefill on f32 caches" : "an hd-512 prefill", sp.base, ws ? ws_bytes : (size_t)0);
        return G4A_EWORKSPACE;
    }
    const bool split = sp.split_tiles > 0 && ws_ok && ws_bytes >= sp.total;
    const bool klo = kv32 && hilo;  // f32 q on f32 caches: K at f32 accuracy as well
    // hd 512: prefill_kernel_w32h for f16 q (its 128 q registers a wave leave no room for
    // the low parts), prefill_kernel_w32d for G4A_Q_HILO
    const bool w32h = HD == 512 && !hilo;
    const prefill_fn fn = HD == 256 ? pick_g<256>(G, out32, hilo, klo, split)
                          : w32h    ? pick_g_w32h(G, out32, split, split || cfg->window > 0)
                                    : pick_g<512>(G, out32, hilo, klo, split);
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
    const int NCOL = prefill_ncol(HD, hilo), BQ = NCOL / G;
    a.n_qblocks = (S + BQ - 1) / BQ;
    if ((int64_t)(start_pos + S) * cfg->n_kv_heads * HD * 2 > 0x7fffffff ||
        (int64_t)S * cfg->n_q_heads * HD * 4 > 0x7fffffff) {
        set_error("q or cache rows beyond 32-bit buffer offsets");
        return G4A_EINVAL;
    }
    a.scale_log2 = cfg->scale * kLog2e;
    a.eps = cfg->eps;
    a.out_q = cfg->out_q;
    a.split_tiles = 0;
    a.max_pieces = 1;
    a.pieces_per_head = 0;
    a.part_o = nullptr;
    a.part_ml = nullptr;
    a.q16 = nullptr;
    a.q16lo = nullptr;
    a.kv_row0 = 0;
    a.kclo = nullptr;
    char* wsp = (char*)ws;  // workspace layout: [K16][V16][K16 low][q16][q16 low][partials][(m, l)]
    if (kv32) {
        const size_t part = sp.kv16_bytes / (klo ? 3 : 2), skip = (size_t)sp.kv_row0 * cfg->n_kv_heads * HD;
        const size_t n8 = (size_t)sp.kv_rows * cfg->n_kv_heads * HD / 8;
        half_t* klo16 = klo ? (half_t*)(wsp + 2 * part) : nullptr;
        hipLaunchKernelGGL(kv16_kernel, dim3((unsigned)((n8 + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                           reinterpret_cast<const float*>(k_cache) + skip, reinterpret_cast<const float*>(v_cache) + skip,
                           (half_t*)wsp, (half_t*)(wsp + part), klo16, n8);
        hipError_t e0 = hipGetLastError();
        if (e0 != hipSuccess) return hip_error(e0, "prefill cache conversion launch");
        a.kc = wsp;
        a.vc = wsp + part;
        a.kclo = klo16;
        a.kv_row0 = sp.kv_row0;
    }
    wsp += sp.kv16_bytes;
    // q in f16 for hd 512 always, for hd 256 when the pieces of a split query block share it
    // (qprep_b's kernel, whose f16 values are those of the hd-256 fused prologue)
    if (HD == 512 || split) {
        const size_t q16b = align256((size_t)S * cfg->n_q_heads * HD * sizeof(half_t));
        half_t* q16 = (half_t*)wsp;
        half_t* q16lo = hilo ? (half_t*)(wsp + q16b) : nullptr;
        const hipError_t e0 = launch_qprep(HD, (long)S * cfg->n_q_heads, (int)cfg->n_q_heads, q, q_gain, rope_cos,
                                           rope_sin, q16, q16lo, cfg->eps, (hipStream_t)stream);
        if (e0 != hipSuccess) return hip_error(e0, "prefill qprep launch");
        a.q16 = q16;
        a.q16lo = q16lo;
        wsp += q16b * (hilo ? 2 : 1);
    }
    // key split (short prompts): pieces of long causal rows, merged by a second kernel
    if (split) {
        a.split_tiles = sp.split_tiles;
        a.max_pieces = sp.max_pieces;
        a.pieces_per_head = sp.total_pieces;
        a.part_o = (half_t*)wsp;
        a.part_ml = (float2*)(wsp + sp.o_bytes);
    }
    a.xcd_runs = a.split_tiles == 0 && cfg->window > 0;
    a.xcd_heads = a.split_tiles == 0 && cfg->window == 0 && 8 % cfg->n_kv_heads == 0 &&
                  ((int64_t)a.n_qblocks * cfg->n_kv_heads) % 8 == 0;
    const dim3 grid = a.split_tiles > 0 ? dim3(sp.total_pieces * cfg->n_kv_heads)
                      : a.xcd_runs || a.xcd_heads ? dim3(a.n_qblocks * cfg->n_kv_heads)
                                        : dim3(a.n_qblocks, cfg->n_kv_heads);
    hipLaunchKernelGGL(fn, grid, dim3(256), 0, (hipStream_t)stream, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_error(e, "prefill launch");
    if (a.split_tiles > 0) {
        auto mf = HD == 256 ? (out32 ? prefill_merge_kernel<float, 256, 128> : prefill_merge_kernel<half_t, 256, 128>)
                  : w32h    ? (out32 ? prefill_merge_kernel<float, 512, 128> : prefill_merge_kernel<half_t, 512, 128>)
                            : (out32 ? prefill_merge_kernel<float, 512, 64> : prefill_merge_kernel<half_t, 512, 64>);
        // one workgroup per 32 columns x 256 dims of a query block
        hipLaunchKernelGGL(mf, dim3(a.n_qblocks, NCOL / 32 * (HD / 256), cfg->n_kv_heads), dim3(256), 0,
                           (hipStream_t)stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return hip_error(e, "prefill merge launch");
    }
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
    const hipError_t e = launch_qprep(HD, rows, (int)cfg->n_q_heads, q, q_gain, rope_cos, rope_sin, (half_t*)q16,
                                      nullptr, cfg->eps, (hipStream_t)stream);
    if (e != hipSuccess) return hip_error(e, "qprep launch");
    return G4A_OK;
}
