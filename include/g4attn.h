/*
 * g4attn.h -- C ABI of the MI355X (gfx950) Gemma 4 E2B attention library
 * (libg4attn.so, built from slang_amd/csrc/).
 *
 * Plain C: pointers, sizes and a config struct; no HIP or torch types. Every
 * pointer argument except `cfg` is DEVICE memory owned by the caller; the
 * library never allocates. `stream` is a hipStream_t passed as void* (NULL =
 * the default stream). Calls are asynchronous on `stream`; argument errors are
 * reported synchronously through the return code before anything is launched.
 *
 * Tensor layouts are the reference runners' (wakoan/slang gemma4_150):
 *   q        [n_tokens][n_q_heads][head_dim]      (runner.py:408-423 outq;
 *                                                  prefill_gpu.py:239 "q" [S][q_dim])
 *   KV cache [position][n_kv_heads][head_dim]     (kernels_dsl.py:1634, 1681 index
 *                                                  ((t*kvH + hKv)*hd + d)), f16 by
 *                                                  default, f32 with G4A_KV_F32
 *   out      [n_tokens][n_q_heads][head_dim]      (attn_101 "out", kernels_dsl.py:1749;
 *                                                  attnh f16, prefill_gpu.py:311-313)
 *   RoPE tables: rows of cos/sin f32 [half] aligned with the call's tokens: row s
 *   belongs to the token at position start_pos+s (prefill, kv write) or to
 *   sequence s's query (decode). Callers offset into their full [max_pos][half]
 *   tables, as the runners pass pre-offset tables to attn_101 (runner.py:283-289)
 *   and absolute tables to the batched kernels (prefill_wgpu.py:142-153).
 *   Pairs i >= the RoPE cutoff are identity rows (cos 1, sin 0) in the tables.
 */
#ifndef G4ATTN_H
#define G4ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* cfg.flags */
#define G4A_KV_F32    0x1u /* caches hold f32 (the reference's own cache type); default f16 */
#define G4A_IN_F16    0x2u /* g4a_kv_write: k/v inputs are f16 (kvnorm_b); default f32 (kvnorm) */
#define G4A_NO_V_NORM 0x4u /* g4a_kv_write, g4a_decode_kv: store v as given instead of RMSNorm(v) */
#define G4A_OUT_F32   0x8u /* g4a_prefill: f32 output (attn_prefill's "out"); default f16 (attnh) */
#define G4A_Q_HILO    0x10u /* g4a_prefill: keep q at f32 accuracy (f16 hi + lo MFMA operands),
                               as attn_prefill's f32 q (kernels_dsl.py:2007-2014); default rounds
                               q to f16 as qprep_b does (kernels_dsl.py:1872-1873) */

typedef struct g4a_cfg {
    uint32_t n_q_heads;  /* qHeads (params[3] of attn_101, params[1] of attn_prefill) */
    uint32_t n_kv_heads; /* kvHeads; n_q_heads % n_kv_heads == 0, group size <= 8 */
    uint32_t head_dim;   /* 256 (sliding layers) or 512 (global layers) */
    uint32_t window;     /* sliding window W; 0 = global (params[5] / params[3]) */
    uint32_t flags;      /* G4A_* */
    float scale;         /* score scale: 1.0 for Gemma 4, 1/sqrt(head_dim) for Gemma 3 */
    float eps;           /* RMSNorm epsilon, 1e-6 in the reference */
    float out_q;         /* SRQ step of the output (attn_101's OUT_Q); 0 = pass-through */
} g4a_cfg;

/* return codes */
#define G4A_OK            0
#define G4A_EINVAL       -1 /* bad argument (null pointer, size, alignment) */
#define G4A_EUNSUPPORTED -2 /* head_dim / group size this build does not instantiate */
#define G4A_EWORKSPACE   -3 /* workspace missing or smaller than the *_ws_bytes size */
#define G4A_EHIP         -4 /* a HIP call failed; g4a_last_error() names it */

const char* g4a_strerror(int code);
/* Detail of the last failure on the calling thread ("" if none). */
const char* g4a_last_error(void);
/*
 * Interface version of the loaded library: G4A_VERSION of the header it was built from.
 *   1  the first release;
 *   2  g4a_gemm_mat.alpha and g4a_norm_in.mult take over what were padding bytes (0 is
 *      read as 1, so zero-initialise both structs); g4a_prefill refuses f32 caches and
 *      head_dim 512 without a workspace (G4A_EWORKSPACE) and keeps K at f32 accuracy on
 *      f32 caches with G4A_Q_HILO; the fused norm prologues refuse x_out / z_out overlapping
 *      their inputs; g4a_qgemv_geglu, g4a_qgemv_gelu_mul, g4a_gemm16_geglu, g4a_geglu16 and
 *      g4a_plegate16 take the layer's GELU table (gelu_lut, before the stream).
 */
#define G4A_VERSION 2
int g4a_version(void);

/*
 * Decode attention: one new query per sequence against its KV cache.
 * Replaces the attn_101 dispatch (gemma4_150/kernels_dsl.py:1537-1749; bound at
 * runner.py:430-441 and metal_runner.py:348-349 with slots
 * [q, q_norm, cos, sin, k, v, partials, out, params]).
 *
 *   key_len[s]  int32, device: keys of sequence s (params[1] keyLen); the query
 *               sits at position key_len[s]-1 (params[2] qOffset = pos).
 *               Sequence s attends keys [max(0, key_len-W), key_len) (W = window, 0 = all).
 *               NULL: every sequence has exactly max_key_len keys, known on the host as
 *               the reference's params are (runner.py:290); the kernel then reads no
 *               length from memory before its first K/V loads.
 *   max_key_len host upper bound of key_len[] (the exact length when key_len is NULL);
 *               sizes the split-KV grid (a tight bound gives the best split).
 *   q           f32 [n_seq][n_q_heads][head_dim], raw: RMSNorm*q_gain then RoPE
 *               are applied in the kernel as attn_101 does (kernels_dsl.py:1593-1615).
 *   q_gain      f32 [head_dim] or NULL (no q RMSNorm).
 *   rope_cos/sin f32 [n_seq][head_dim/2] for each query's position, or NULL (no RoPE).
 *   k_cache/v_cache sequence s at base + s*seq_stride elements, rows [pos][kvH][hd].
 *   out         f32 [n_seq][n_q_heads][head_dim] (srq'd with out_q when nonzero).
 *   ws          workspace of at least g4a_decode_ws_bytes() bytes (256-byte aligned) for
 *               the split partials (acc, m, l) that attn_101 keeps in `partials`; it needs
 *               no initialisation. Long sequences are split over workgroups and merged by a
 *               second kernel on the same stream. Concurrent calls need distinct ws.
 */
size_t g4a_decode_ws_bytes(const g4a_cfg* cfg, int n_seq, int max_key_len);
int g4a_decode(const g4a_cfg* cfg, int n_seq, int max_key_len, const int32_t* key_len,
               const float* q, const float* q_gain, const float* rope_cos, const float* rope_sin,
               const void* k_cache, const void* v_cache, int64_t seq_stride, float* out,
               void* ws, size_t ws_bytes, void* stream);

/*
 * Decode step with its KV write fused in: the kvnorm dispatch (kernels_dsl.py:573-618,
 * bound at runner.py:424-429) and the attn_101 dispatch that follows it
 * (runner.py:430-441) as one call. For every sequence s with key_len[s] > 0 the raw rows
 * k_new/v_new [n_seq][n_kv_heads][head_dim] (f32, the q/k/v projection's output) are
 * prepared exactly as g4a_kv_write prepares them (srq with k_in_q / v_in_q, k RMSNorm *
 * k_gain then RoPE with the sequence's rope_cos/rope_sin row -- the query's position --,
 * v RMSNorm unless G4A_NO_V_NORM) and stored at row key_len[s]-1 of the caches; the
 * attention then includes that row. The workgroup whose split holds the new key writes
 * it, so the row costs no extra kernel. Other arguments, the workspace and the result
 * are those of g4a_decode; the caches are written, so they are not const here.
 */
int g4a_decode_kv(const g4a_cfg* cfg, int n_seq, int max_key_len, const int32_t* key_len,
                  const float* q, const float* q_gain, const float* rope_cos, const float* rope_sin,
                  const float* k_new, const float* v_new, float k_in_q, float v_in_q,
                  const float* k_gain, void* k_cache, void* v_cache, int64_t seq_stride, float* out,
                  void* ws, size_t ws_bytes, void* stream);

/*
 * g4a_decode without a workspace: no counterpart in the reference (whose runners own a
 * persistent `partials` buffer). It is for callers that cannot allocate device memory --
 * code under HIP graph capture, serving loops or harnesses that forbid hipMalloc. The
 * split partials live in a device array inside the library, G4A_DECODE_SCRATCH_BYTES per
 * GPU, held from the library's load until the process ends; the call allocates nothing.
 * Arguments, kernels and results are those of g4a_decode (bit-identical for the same
 * inputs). A call whose partials need more than the array holds (g4a_decode_ws_bytes >
 * G4A_DECODE_SCRATCH_BYTES: roughly n_seq * n_kv_heads * splits * G * head_dim * 4 bytes)
 * returns G4A_EWORKSPACE before launching. The stream must belong to the current device.
 * Every call on one GPU shares that GPU's array, so calls that overlap on one GPU (two
 * streams, two threads) race: serialise them, or use g4a_decode with distinct workspaces.
 */
#define G4A_DECODE_SCRATCH_BYTES (8u << 20)
int g4a_decode_noalloc(const g4a_cfg* cfg, int n_seq, int max_key_len, const int32_t* key_len,
                       const float* q, const float* q_gain, const float* rope_cos, const float* rope_sin,
                       const void* k_cache, const void* v_cache, int64_t seq_stride, float* out,
                       void* stream);

/*
 * Batched causal prefill attention for S tokens at positions start_pos..start_pos+S-1.
 * Replaces PrefillGPU._attn_gemm (prefill_gpu.py:259-313: qprep_b -> QK^T GEMM ->
 * smax_b -> PV GEMM -> attnout_b) and the fused attn_prefill dispatch
 * (kernels_dsl.py:1950-2098, bound at prefill_gpu.py:347-354 with slots
 * [q, q_norm, cosT, sinT, k, v, out, (startPos, qH, kvH, W, S)]).
 *
 *   q        f32 [S][n_q_heads][head_dim] raw; RMSNorm*q_gain + RoPE are applied in
 *            the kernel and the result is rounded to f16 (qprep_b, kernels_dsl.py:1872-1873).
 *   rope_cos/sin f32 [S][head_dim/2] rows for the S positions, or NULL.
 *   k_cache/v_cache rows [0, start_pos+S) already written (g4a_kv_write).
 *   out      f16 [S][n_q_heads][head_dim] (attnh), or f32 with G4A_OUT_F32.
 *   Token s attends keys [max(0, p+1-W), p] with p = start_pos+s (kernels_dsl.py:1986-1992).
 *   ws/ws_bytes: workspace of g4a_prefill_ws_bytes() bytes (256-byte aligned) for the
 *            key split of short prompts: long causal rows are then spread over several
 *            workgroups and merged by a second kernel on the same stream. It needs no
 *            initialisation. With ws NULL or smaller, the call runs unsplit (same results
 *            up to summation order, slower); ws_bytes() is 0 when no split would be used.
 */
size_t g4a_prefill_ws_bytes(const g4a_cfg* cfg, int S, int start_pos);
int g4a_prefill(const g4a_cfg* cfg, int S, int start_pos, const float* q, const float* q_gain,
                const float* rope_cos, const float* rope_sin, const void* k_cache,
                const void* v_cache, void* out, void* ws, size_t ws_bytes, void* stream);

/*
 * q RMSNorm*q_gain + RoPE for S*n_q_heads rows, stored f16 [S][n_q_heads][head_dim].
 * Replaces qprep_b (kernels_dsl.py:1837-1873, dispatched at prefill_gpu.py:283-285 with
 * slots [q, q_norm, cosT, sinT, qf16, (startPos, qHeads)]). Uses the same arithmetic and
 * lane layout as g4a_prefill's prologue, so it yields exactly the f16 q g4a_prefill
 * feeds its MFMAs (without G4A_Q_HILO). rope_cos/sin: [S][head_dim/2] rows or NULL.
 */
int g4a_qprep(const g4a_cfg* cfg, int S, const float* q, const float* q_gain,
              const float* rope_cos, const float* rope_sin, void* q16, void* stream);

/*
 * KV-cache write of S new tokens at rows start_pos..start_pos+S-1:
 *   k <- RoPE(RMSNorm(srq(k, k_in_q)) * k_gain),  v <- RMSNorm(srq(v, v_in_q)) (no gain).
 * Replaces kvnorm (kernels_dsl.py:573-618, dispatched at runner.py:424-429 with slots
 * [outk, outv, k_norm, cos, sin, kc, vc, pkv]) and kvnorm_b (kernels_dsl.py:1789-1834,
 * prefill_gpu.py:335-342, slots [kraw, vraw, k_norm, cosT, sinT, kc, vc, (startPos, kS, vS)]).
 *
 *   k, v     [S][n_kv_heads][head_dim], f32 (kvnorm) or f16 with G4A_IN_F16 (kvnorm_b).
 *   k_gain   f32 [head_dim] or NULL (no k RMSNorm). G4A_NO_V_NORM skips the v norm.
 *   rope_cos/sin f32 [S][head_dim/2] or NULL.
 *   k_cache/v_cache rows of [pos][kvH][hd], f16 (or f32 with G4A_KV_F32).
 */
int g4a_kv_write(const g4a_cfg* cfg, int S, int start_pos, const void* k, const void* v,
                 float k_in_q, float v_in_q, const float* k_gain, const float* rope_cos,
                 const float* rope_sin, void* k_cache, void* v_cache, void* stream);

/*
 * ---- The q/k/v producer: projections with QAT weights --------------------------------
 * Packed weights: row o of an [n_out][n_in] matrix is n_in*bits/32 uint32 words; value i
 * of the row sits at bit 8*(i/(8/bits)) + bits*(i%(8/bits)) of the row's bytes (byte-major,
 * low bits first) and stands for row_scale[o] * (q - 2^(bits-1)) (dq_f16,
 * kernels_dsl.py:2101-2138; qkv_70 unpacks the 4-bit case the same way, :1421-1426).
 */
/*
 * Dequantise to f16: out[o][i] = f16(w_scale[o] * (q - 2^(bits-1))), the product in f32.
 * Replaces dq_f16 (kernels_dsl.py:2101-2138; PrefillGPU._dq, prefill_gpu.py:186-200, slots
 * [bits, scale(+offset), dst, (n_in, n_out)]). bits 2, 4 or 8; n_in a multiple of 128/bits.
 * Weights are static: run it once per layer at load, or per call as the reference does.
 */
int g4a_dequant(int bits, int n_in, int n_out, const uint32_t* w_bits, const float* w_scale,
                void* out_f16, void* stream);
/*
 * Decode q/k/v projections of one token, 4-bit QAT rows. Replaces qkv_70
 * (kernels_dsl.py:1384-1480, dispatched at runner.py:408-423 with slots [a, q_bits, k_bits,
 * v_bits, scales, sum_a, out_q, out_k, out_v, (q_out, k_out, v_out)]):
 *   out_q[o] = srq(scales[o] * (sum_i q[o][i] a[i] - 8 sum_a), q_out)            o < q_dim
 *   out_k[o] = srq(scales[q_dim + o] * (... k rows ...), k_out)                   o < kv_dim
 *   out_v[o] = srq(scales[q_dim + kv_dim + o] * (... v rows ...), v_out)
 *   a f32 [hidden] (hidden a multiple of 32, <= 4096); sum_a f32 [1] = sum of a, as
 *   rmssrq_69 leaves it; q_dim, kv_dim multiples of 8. kv_dim 0 = a KV-sharing layer:
 *   q only, k/v pointers unused (runner.py:416-419).
 */
int g4a_qkv_gemv(int hidden, int q_dim, int kv_dim, const float* a, const float* sum_a,
                 const uint32_t* q_bits, const uint32_t* k_bits, const uint32_t* v_bits,
                 const float* scales, float q_out, float k_out, float v_out, float* out_q,
                 float* out_k, float* out_v, void* stream);
/*
 * srqh_b (kernels_dsl.py:232-242; prefill_gpu.py:286-288, :327-334): out_f16[i] =
 * f16(srq(a[i], a_in_q)), 0 = convert only. n a multiple of 8. The activation operand of
 * g4a_gemm16, made once and shared by the q, k and v products of a layer.
 */
int g4a_srqh(int n, const float* a, float a_in_q, void* out_f16, void* stream);

/* One product of g4a_gemm16: out = A . w^T, w f16 [n][K] (g4a_dequant's output); out f16
 * [M][n] = f16(f32-accumulated sum) as gemm_tiled writes it (kernels_dsl.py:34-136), or
 * with out_f32 != 0 f32 [M][n] = srq(f32(that f16), out_q), srq_b's q path (:246-255). */
typedef struct {
    const void* w_f16;
    void* out;
    int n;        /* rows of w = output columns, a multiple of 128 */
    int out_f32;
    float out_q;
    float alpha;  /* the f16 result is f16(alpha * sum), gemm_tiled's alpha (kernels_dsl.py:96-103;
                     the down projection's down_in, prefill_gpu.py:377); 0 means 1 */
} g4a_gemm_mat;

/*
 * Up to three GEMMs sharing the f16 activation A [M][K] in one launch: the q, k and v
 * projection GEMMs of PrefillGPU._layer (prefill_gpu.py:327-342, each a _gemm on srqh_b's
 * output) as one dispatch. K a multiple of 64.
 */
int g4a_gemm16(int M, int K, const void* a_f16, int n_mats, const g4a_gemm_mat* mats, void* stream);

/*
 * g4a_gemm16 with a workspace, which lets a launch with too few output tiles to fill the
 * GPU (the N 1536 products of the decoder prefill, the narrow per-layer-embedding gate)
 * split K over several workgroups per tile. Replaces the same dispatches as g4a_gemm16
 * (gemm_tiled, kernels_dsl.py:34-136, from PrefillGPU._gemm / _gemm_dsl, prefill_gpu.py:151-184);
 * the workspace plays the part of the scratch PrefillGPU sizes per prompt (_alloc_acts,
 * prefill_gpu.py:229-256).
 * Each split's f32 partial tile goes to the workspace and the tile's last workgroup adds them
 * in split order, so the result is deterministic and each output is still f16(alpha * sum)
 * of one f32 sum (its terms grouped by K range). ws: device memory of at least
 * g4a_gemm16_ws_bytes(...) bytes (0: the launch does not split, ws may be NULL), 256-byte
 * aligned; its first G4A_GEMM_TICKET_BYTES bytes are per-tile tickets that must be zero before
 * the first call on it (every call leaves them zero), the rest needs no initialisation. Calls
 * that may run concurrently need separate workspaces. Returns G4A_EWORKSPACE if ws_bytes is
 * short.
 */
/*
 * The MLP's gate and up GEMMs and geglu_b in one launch: the two _gemm dispatches on the
 * pre-FFN operand and the geglu_b dispatch after them (prefill_gpu.py:365-371; geglu_b,
 * kernels_dsl.py:259-290). out f16 [M][n] = geglu_b's code of g = f16(A . w_gate^T) and
 * u = f16(A . w_up^T): f16(clamp(round(gelu(srq(g, gate_q)) * srq(u, up_q) / out_q), -128,
 * 127)), or f16(gelu(..) * ..) when out_q is 0 -- the same values as g4a_gemm16 on the two
 * matrices followed by g4a_geglu16, without writing or reading g and u. w_gate and w_up are
 * f16 [n][K]; K and n multiples of 64. gelu_lut as for g4a_geglu16.
 */
int g4a_gemm16_geglu(int M, int K, const void* a_f16, const void* w_gate_f16, const void* w_up_f16, int n,
                     float gate_q, float up_q, float out_q, void* out_f16, const float* gelu_lut, void* stream);

#define G4A_GEMM_TICKET_BYTES 2048
size_t g4a_gemm16_ws_bytes(int M, int K, int n_mats, const g4a_gemm_mat* mats);
int g4a_gemm16_ws(int M, int K, const void* a_f16, int n_mats, const g4a_gemm_mat* mats, void* ws,
                  size_t ws_bytes, void* stream);

/*
 * ---- The rest of a decode step: the decoder layer around the attention block ---------
 * One token's layer (gemma4_150/reference.py:141-191) is, with x f32 [H]:
 *   a = srq(rms(x, in_norm), qkv_in)        g4a_rms_norm (out2, sum2)     rmssrq_69
 *   q/k/v, KV write, attention              g4a_qkv_gemv, g4a_decode_kv   qkv_70, kvnorm, attn_101
 *   x = x + rms(qlin(attn, o), post_attn)   g4a_qgemv, g4a_rms_norm       oproj_73
 *   y2 = f16(srq(f16(rms(x, pre_ffn)), gate_in))  g4a_rms_norm (f16_2)
 *   x = x + rms(qlin(srq(gelu(qlin(y2, gate)) * qlin(y2, up), down_in), down), post_ffn)
 *                                           g4a_qgemv, g4a_geglu          gateup_74/95, down_75/96
 *   x = (x + rms(ilin(gelu(ilin(x, plegate)) * ple_in[L], pleproj), post_ple)) * layer_scalar
 *                                           g4a_qgemv (8-bit), g4a_geglu  plegate_76, pleproj_77
 * and around the layers (reference.py:114-139, 193-207): the token and per-layer
 * embedding rows (g4a_embed; embed_00, plegather_01), the per-layer-input projection
 * (g4a_gemv_f16 + g4a_rms_norm), the final norm, the 2-bit lm_head (g4a_qgemv) and the
 * softcap + greedy argmax (g4a_softcap_argmax; logits_33, argmax1_34/argmax2_35).
 */
/*
 * Quantised GEMV: out[o] = srq(w_scale[o] * sum_i (q[o][i] - 2^(bits-1)) * srq(x[i], in_q), out_q)
 * (reference.py:96-101 _qlin; :103-111 _ilin_raw is the bits = 8 case over export.py's
 * biased codes, :150-156; :200-206 the lm_head with in_q = out_q = 0). Rows are packed as
 * for g4a_dequant; bits 2, 4 or 8; n_in a multiple of 128/bits. x f32 [n_in], 16-byte
 * aligned; out f32 [n_out]. With in_q > 0 and 4/8-bit rows of at most 64 16-byte chunks
 * (or a norm prologue, in the fused GEMVs below) the row sum is formed in int32 over srq's
 * grid index of x, exactly at any row length: out = srq(f32(f32(D) * in_q) * w_scale, out_q),
 * D = sum (q - zp) * clamp(rint(x / in_q)), rounded to f32 once; the f32 accumulation of the
 * reference rounds its partial sums, so the two can differ in the last bits before the output
 * srq.
 */
int g4a_qgemv(int bits, int n_in, int n_out, const float* x, float in_q, const uint32_t* w_bits,
              const float* w_scale, float out_q, float* out, void* stream);
/*
 * Optional norm prologue of the fused GEMVs below: the residual add and norm(s) in front of
 * them, done by every workgroup while it stages x (the runner's kernels fuse them the same
 * way, oproj_73 ending with the pre-FFN norm, pleproj_77 with the next layer's input norm),
 * so no kernel of its own runs:
 *   x = (res + a / sqrt(mean(a^2) + eps) * w1) * mult  (stored to x_out by one workgroup)
 *   z = x / sqrt(mean(x^2) + eps) * w2, or z = x when w2 is NULL
 *   GEMV input = f16 ? f16(srq(f16(z), q2)) : srq(z, q2)   (stored to z_out if non-NULL)
 * n_in <= 2048; x_out must not alias a, res or w1 (other workgroups still read them).
 * mult is the layer scalar of the per-layer-embedding add (reference.py:191); 0 is read as 1,
 * so a zero-initialised struct leaves x unscaled.
 */
typedef struct {
    const float* a;
    const float* res;
    const float* w1;
    const float* w2;
    float* x_out;
    float* z_out;
    float q2;
    int f16;
    float eps;
    float mult;
} g4a_norm_in;
/*
 * GELU of an srq'd value: gelu_lut, when given, is the layer's 256-entry table of the srq grid
 * the value sits on, lut[k + 128] = f32(gelu_tanh(k * step)) evaluated in float64 -- the
 * exported L{L}.gelu_gate / L{L}.gelu_plegate (export.py:30-33, :150, :161) -- and GELU of a
 * grid value v is lut[clamp(round(v / step), -128, 127) + 128], as every runner kernel forms it
 * (geglu_b kernels_dsl.py:283, plegate_76 :867, gateup_74/95 :1292/:1373, plegate_b :1785). NULL
 * (or a zero step) computes gelu_tanh in f32 instead (reference.py:34-35).
 *
 * The MLP's gate/up pair with its GeGLU in one pass over x (gateup_74/95; reference.py:176-181):
 *   out[o] = srq(gelu(g[o]) * u[o], out_q),
 *   g = the g4a_qgemv output of the gate rows (gate_in_q, gate_out_q), u that of the up rows;
 *   gelu_lut: the table of the gate_out_q grid (L{L}.gelu_gate) or NULL.
 */
int g4a_qgemv_geglu(int bits, int n_in, int n_out, const float* x, const uint32_t* gate_bits,
                    const float* gate_scale, float gate_in_q, float gate_out_q, const uint32_t* up_bits,
                    const float* up_scale, float up_in_q, float up_out_q, float out_q, float* out,
                    const g4a_norm_in* pro, const float* gelu_lut, void* stream);
/* g4a_qgemv with the per-layer-embedding gate's epilogue: out[o] = gelu(y[o]) * mul[o]
 * (plegate_76; reference.py:186-187, mul = the layer's per-layer input). pro as above;
 * gelu_lut the table of the out_q grid (L{L}.gelu_plegate) or NULL. */
int g4a_qgemv_gelu_mul(int bits, int n_in, int n_out, const float* x, float in_q, const uint32_t* w_bits,
                       const float* w_scale, float out_q, const float* mul, float* out,
                       const g4a_norm_in* pro, const float* gelu_lut, void* stream);
/*
 * g4a_qkv_gemv with its input made in the kernel from the previous layer's tail, so the
 * layer-end add and the next input norm (rmssrq_69 after pleproj_77, runner.py:373-407)
 * need no launch of their own: every workgroup forms
 *   x = (res + a_pre / sqrt(mean(a_pre^2) + eps) * w1) * mult,  a = srq(rms(x) * w2, q2)
 * from pro (w2 required, f16 must be 0) and runs qkv_70 on a with
 * sum_a = sum of a. One workgroup stores x to pro->x_out, a to pro->z_out and sum_a to
 * sum_out (each may be NULL). hidden <= 2048.
 */
int g4a_qkv_gemv_norm(int hidden, int q_dim, int kv_dim, const g4a_norm_in* pro, float* sum_out,
                      const uint32_t* q_bits, const uint32_t* k_bits, const uint32_t* v_bits,
                      const float* scales, float q_out, float k_out, float v_out, float* out_q,
                      float* out_k, float* out_v, void* stream);
/* Dense f16 GEMV: out[o] = sum_i w[o][i] x[i] in f32 (the per-layer-input projection,
 * reference.py:136, exported f16 by export.py:95). n_in a multiple of 8. */
int g4a_gemv_f16(int n_in, int n_out, const float* x, const void* w_f16, float* out, void* stream);
/*
 * RMSNorm family over n_rows rows of n values (reference.py:38-43 and the sandwich adds
 * of :170, :183, :191; :133-139 for the per-layer-input context):
 *   y = x' / sqrt(mean(x'^2) + eps) * w (w NULL: no gain), x' = x * pre
 *   out = (res + y) * mult (res NULL: 0)
 *   z = out, or with w2 the next norm z = out / sqrt(mean(out^2) + eps) * w2 (the pre-FFN
 *   norm after the o_proj add, the next layer's input norm after the layer's last add)
 *   out2 = srq(z, q2), or with f16_2 f16(srq(f16(z), q2)) (reference.py:176-178);
 *   sum2[row] = sum of out2 (qkv_70's sum_a). w2, out2 and sum2 may be NULL.
 * out may alias res (not x).
 */
int g4a_rms_norm(int n_rows, int n, const float* x, float pre, const float* w, const float* res,
                 float mult, float eps, float* out, const float* w2, float q2, int f16_2, float* out2,
                 float* sum2, void* stream);
/* out[i] = srq(gelu_tanh(a[i]) * b[i], out_q) (reference.py:34-35, :181, :188). */
int g4a_geglu(int n, const float* a, const float* b, float out_q, float* out, void* stream);
/*
 * Embedding row of the token id tok[0] (device memory, so a step can take the previous
 * step's argmax): out[j] = mult * row_scale[tok * (n/group) + j/group] * (code_j - 2^(bits-1))
 * from row tok of a packed table of n_rows rows (reference.py:114-121 embed: 2-bit, group
 * n; :123-131 ple_table: 4-bit, group ple_d). An id outside [0, n_rows) gives zeros.
 */
int g4a_embed(int bits, int n, const void* table, int64_t n_rows, const int32_t* tok,
              const float* row_scale, int group, float mult, float* out, void* stream);
/* g4a_embed for n_tok tokens tok[0..n_tok) into out [n_tok][n]: embed_00 and plegather_01 over
 * the S tokens of a batched prefill (kernels_dsl.py:433-479; prefill_gpu.py:412-420). */
int g4a_embed_rows(int bits, int n, const void* table, int64_t n_rows, const int32_t* tok, int n_tok,
                   const float* row_scale, int group, float mult, float* out, void* stream);
/* logits <- cap * tanh(logits / cap) in place (cap 0: unchanged) and tok[0] = the first
 * index of the maximum (reference.py:207; runner.py:501-505 argmax1_34 -> argmax2_35 on the
 * GPU). ws: g4a_softcap_argmax_ws_bytes(n) bytes for the per-workgroup candidates; logits
 * 16-byte aligned. */
size_t g4a_softcap_argmax_ws_bytes(int n);
int g4a_softcap_argmax(int n, float* logits, float cap, int32_t* tok, void* ws, size_t ws_bytes,
                       void* stream);

/*
 * ---- The layers-outer batched prefill around the attention block ----------------------
 * PrefillGPU._layer (gemma4_150/prefill_gpu.py:316-395) over S token rows: the f16 GEMMs are
 * g4a_gemm16 on dequantised weights (g4a_dequant), the attention g4a_prefill, and the tails
 * between them these three.
 */
/* g4a_rows_tail modes: the next GEMM's f16 operand y16 made from the updated row */
#define G4A_TAIL_NONE   0 /* no y16 */
#define G4A_TAIL_SRQ    1 /* y16 = f16(srq(hidden, q2))                          srqh_b */
#define G4A_TAIL_NORM   2 /* y16 = f16(srq(rms(hidden) * w2, q2))                rmssrq_69 + srqh_b */
#define G4A_TAIL_NORM16 3 /* y16 = f16(srq(f32(f16(rms(hidden) * w2)), q2))      rmssrqh_b */
/*
 * Per row r of n values (n <= 4096): when x16 is given, the residual add + RMSNorm of rmsadd_b
 * (kernels_dsl.py:622-657; prefill_gpu.py:364, 378, 389):
 *   d = srq(f32(x16[r]), x_q);  hidden[r] = (hidden[r] + d / sqrt(mean(d^2) + eps) * w1) * mult
 * then y16[r] by mode, rms(h) = h / sqrt(mean(h^2) + eps) (rmssrqh_b :660-710, srqh_b :233-242,
 * rmssrq_69 :158-206). x16 NULL: no add, y16 from hidden as it is (the input norm of layer 0,
 * prefill_gpu.py:430-431). hidden f32 [n_rows][n], x16/y16 f16 [n_rows][n].
 */
int g4a_rows_tail(int n_rows, int n, const void* x16, float x_q, const float* w1, float mult, float eps,
                  float* hidden, int mode, const float* w2, float q2, void* y16, void* stream);
/*
 * geglu_b (kernels_dsl.py:259-290; prefill_gpu.py:373-375) over n values (a multiple of 8):
 *   y = gelu(srq(f32(gate16), gate_q)) * srq(f32(up16), up_q)
 *   out16 = f16(clamp(round(y / out_q), -128, 127)) -- the code on out_q's grid, which the down
 *   GEMM scales back with alpha = out_q --, or f16(y) when out_q is 0.
 * gelu_lut: the table of the gate_q grid (L{L}.gelu_gate; see g4a_qgemv_geglu) or NULL.
 */
int g4a_geglu16(int n, const void* gate16, const void* up16, float gate_q, float up_q, float out_q,
                void* out16, const float* gelu_lut, void* stream);
/*
 * plegate_b then srqh_b (kernels_dsl.py:1767-1786, 233-242; prefill_gpu.py:381-384) over n_rows
 * rows of d values (a multiple of 8):
 *   out16[s][o] = f16(srq(gelu(srq(f32(lin16[s][o]), lin_q)) * ple[s * ple_stride + o], out_q))
 * ple: the layer's slice of the per-layer inputs [S][nL][d] (ple_stride = nL * d); gelu_lut the
 * table of the lin_q grid (L{L}.gelu_plegate; see g4a_qgemv_geglu) or NULL.
 */
int g4a_plegate16(int n_rows, int d, const void* lin16, float lin_q, const float* ple, int ple_stride,
                  float out_q, void* out16, const float* gelu_lut, void* stream);

/*
 * ---- Roofline probes (measurement only; no counterpart in the reference) ------------------
 * The denominators the kernels above are measured against, taken on the GPU they run on.
 * sink: device memory of g4a_probe_sink_bytes() bytes that receives values derived from the
 * work (so none of it is dead); its contents mean nothing.
 *   g4a_probe_read  reads bytes (a multiple of 4096, at most 2 GiB) from p once, with 16-byte
 *                   non-temporal loads over `workgroups` workgroups of 256 threads (0: 2048,
 *                   at most 4096): the best any kernel reading that much from HBM can do.
 *   g4a_probe_mfma  `workgroups` workgroups of 512 threads (at most 4096), each wave issuing
 *                   8 * iters v_mfma_f32_32x32x16_f16 (32768 FLOP each) from registers, with
 *                   8 independent accumulator chains: the reachable dense f16 MFMA rate.
 */
size_t g4a_probe_sink_bytes(void);
int g4a_probe_read(const void* p, size_t bytes, int workgroups, void* sink, void* stream);
int g4a_probe_mfma(int workgroups, int iters, void* sink, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* G4ATTN_H */
