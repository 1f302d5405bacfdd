/* t2r.h -- C-ABI of the MI355X-native W8A8 decoder datapath (libt2r.so, gfx950).
 *
 * The drop-in boundary for the path jonathansong/Torch2RISCV-accelerator runs on its FPGA
 * accelerator and models on the CPU (llm/ref_model.py DeviceModel, llm/sa_funcsim.py,
 * llm/sfu.py, llm/fp32.py). Two levels, as llm/runtime.py dispatches:
 *   - op level: one call per piece of the reference's token list (ModelCompiler's embed,
 *     rmsnorm, quant_act + W8A8 linear, rope, kv_append, attention, silu_mul / ffn_up,
 *     residual, final: llm/compile_model.py:147-349), each step for step the DeviceModel
 *     method it names;
 *   - model level: one decode step / one prefill of a resident model, the per-token
 *     Device.submit + wait of llm/runtime.py:107-125.
 *
 * Conventions
 *   - Tensor arguments are DEVICE pointers owned by the caller; the library never allocates,
 *     frees or synchronises on these calls. Every call enqueues on `stream` (a hipStream_t
 *     passed as void*, NULL = the default stream) and returns T2R_OK, or a negative code
 *     BEFORE launching anything when an argument is invalid (the reference's SaError shape /
 *     range checks, llm/sa_funcsim.py:26-31, as T2R_ESHAPE / T2R_ERANGE).
 *   - Numerics: int8 x int8 -> exact int32; y = F(F(f32(acc) * s_w) * s_x); fp32 vector steps
 *     with one IEEE rounding each, never fused; EXP / RECIP / RSQRT bit-exact with the SFU;
 *     sums in the D-lane order (D = 8 or 16). Results are bit-identical to the reference's.
 *   - Matrices are row-major; linear weights are (out, in) int8 with one fp32 scale per row.
 *   - Thread safety: calls on different streams may run concurrently; the only global state
 *     is the SFU table constant, written once per device by the first call (t2r_init).
 */
#ifndef T2R_H
#define T2R_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define T2R_ABI_VERSION 2

enum {
  T2R_OK = 0,
  T2R_EINVAL = -1,   /* null pointer, bad enum, bad config                             */
  T2R_ESHAPE = -2,   /* a size the kernels cannot take (~ SaError XERR_SHAPE = 1)       */
  T2R_ERANGE = -3,   /* an index or size out of range (~ SaError XERR_RANGE = 2)        */
  T2R_EHIP = -4,     /* a HIP runtime error (launch or symbol copy)                     */
  T2R_ENOMEM = -5,   /* the workspace given is too small                                */
  T2R_ESTATE = -6    /* a model handle in the wrong state                               */
};

int t2r_abi_version(void);
const char* t2r_strerror(int code);
/* Writes the SFU tables (llm/sfu.py:42-56) to the current device; the other calls do it
 * themselves on first use. Returns T2R_OK or T2R_EHIP. */
int t2r_init(void);
/* Copies the SFU tables as the device holds them: T/S of EXP (64 + 64), RECIP (64 + 64),
 * RSQRT (128 + 128) as fp32 bit patterns into host memory out[512]. */
int t2r_sfu_tables(uint32_t* out);

/* ---------------------------------------------------------------- element-wise hooks */
/* fn 0 EXP, 1 RECIP, 2 RSQRT, 3 ABS on n fp32 bit patterns (llm/sfu.py:69-118). */
int t2r_sfu(int fn, const uint32_t* x, uint32_t* y, int64_t n, void* stream);
/* Self-check of the datapath SFU (no counterpart in the reference; for tests): every fp32 input
 * x in [first, first + count) (as bit patterns, count <= 2^32 - first) through fn (0 EXP,
 * 1 RECIP, 2 RSQRT, 3 the softmax's EXP on its domain x <= 0 and NaN, 4 the gates' RECIP on its
 * domain x >= 1 and NaN, 5 the softmax's EXP under a finite maximum on its domain x <= 0, 6 the
 * gates' pair-table EXP on every non-NaN x, 7 the gates' pair-table RECIP on x >= 1 (not NaN);
 * other inputs of fn 3 .. 7 skipped) as the kernels compute it and as the literal per-operation FTZ
 * sequence of llm/sfu.py:69-118 (EXP for fn 3, 5 and 6, RECIP for fn 4 and 7). Device
 * out[0] = number of inputs whose results differ, out[1] = the smallest such input (0xFFFFFFFF if
 * none). */
int t2r_sfu_check(int fn, uint64_t first, uint64_t count, uint32_t* out, void* stream);
/* The fp32 primitives (llm/fp32.py:78-189): op 0 add, 1 sub, 2 mul (flush-to-zero), 3 ldexp
 * (b = int32 exponents), 4 floor to int32 (saturated), 5 to_i8 (RNE, +-127, NaN -> 0),
 * 6 int32 -> fp32 (RNE), 7 IEEE mul, 8 IEEE add (the vector steps). */
int t2r_fp32_op(int op, const uint32_t* a, const uint32_t* b, uint32_t* y, int64_t n, void* stream);
/* Integer REQUANT of the vector engine (llm/sa_funcsim.py:265-274, driver/pynq_matmul.py:127-135):
 * out = sat8(clamp(((r * scale + 2^(shift-1)) >> shift) + zp, lo, hi)); scale is signed 16-bit. */
int t2r_requant(const int32_t* r, int64_t n, int scale, int shift, int zp, int lo, int hi, int8_t* out,
                void* stream);

/* ---------------------------------------------------------------- op level */
/* x[r] = F(f32(emb_q[tokens[r]]) * emb_s[tokens[r]]) (llm/ref_model.py:221; ModelCompiler.embed
 * llm/compile_model.py:192-201). A token outside [0, vocab) reads row 0 and sets *status = 1
 * (status may be NULL). */
int t2r_embed(const int8_t* emb_q, const float* emb_s, const int32_t* tokens, int rows, int dim, int vocab,
              float* x, int32_t* status, void* stream);
/* RMSNorm of rows x[rows, n] (DeviceModel.rmsnorm llm/ref_model.py:204-207; ModelCompiler.rmsnorm
 * llm/compile_model.py:147-156); n <= 8192. */
int t2r_rmsnorm(const float* x, const float* g, int rows, int n, float eps, int D, float* out, void* stream);
/* Per-row dynamic int8 (DeviceModel.quant_act llm/ref_model.py:191-196; CL.quant_act
 * llm/compile_layer.py:66-77); n <= 8192, n % 16 == 0. */
int t2r_quant_act(const float* x, int rows, int n, int8_t* xq, float* s_x, void* stream);
/* The W8A8 linear layer of one activation row (DeviceModel.linear llm/ref_model.py:198-202;
 * SaFuncSim.gemv llm/sa_funcsim.py:138-162; CL.linear llm/compile_layer.py:93-182):
 * acc[n] = sum_k xq[k] w[n, k] (int32), y[n] = F(F(f32(acc) * s_w[n]) * s_x[0]) (+ residual[n]
 * first rounded sum, llm/compile_model.py:330-331). y is required; acc_out (the int32 sums, a parity
 * hook) and residual may be NULL; residual may alias y. K % 16 == 0, K <= 8192. */
int t2r_gemv_w8a8(const int8_t* w, const float* s_w, const int8_t* xq, const float* s_x, int N, int K, float* y,
                  int32_t* acc_out, const float* residual, void* stream);
/* The same over M activation rows xq[M, K] with scales s_x[M] (prefill rows,
 * compiler/plugins/sa/transforms/SahlExpandKernels.cpp:205 expandLinearRows) on int8 MFMA;
 * y, acc_out and residual are [M, N]. */
int t2r_gemm_w8a8(const int8_t* w, const float* s_w, const int8_t* xq, const float* s_x, int M, int N, int K,
                  float* y, int32_t* acc_out, const float* residual, void* stream);
/* RoPE of rows v[rows, n] in place at positions pos[rows] (DeviceModel.rope llm/ref_model.py:209-214;
 * ModelCompiler.rope llm/compile_model.py:203-214): pairs (2i, 2i+1), tables [S, half] with
 * half = head_dim / 2, pair i using column i % half. A row whose position is outside [0, S) is
 * left unchanged. */
int t2r_rope(float* v, const float* cos_t, const float* sin_t, const int32_t* pos, int rows, int n, int half, int S,
             void* stream);
/* KV append (llm/ref_model.py:228-229; ModelCompiler.kv_append llm/compile_model.py:221-231):
 * kc[pos[r]] = to_i8(F(k[r] * inv_sk)), vc[pos[r]] = to_i8(F(v[r] * inv_sv)); caches [S, kv_dim].
 * A row whose position is outside [0, S) is not written. */
int t2r_kv_append(const float* k, const float* v, float inv_sk, float inv_sv, int8_t* kc, int8_t* vc,
                  const int32_t* pos, int rows, int kv_dim, int S, void* stream);
/* Attention of rows q[rows, H * hd] (already rotated) at positions pos[rows] over the int8 cache
 * rows 0..pos (DeviceModel.forward llm/ref_model.py:230-243; ModelCompiler.attention
 * llm/compile_model.py:233-293; GQA: compiler/frontend/qhf.py:304-319). a_k = F(s_k / sqrt(hd)),
 * a_v = F(s_v / 127). S = cache rows <= 8192, hd <= 128 and a multiple of 8. */
int t2r_attn_decode(const float* q, const int8_t* kc, const int8_t* vc, const int32_t* pos, int rows, int H,
                    int Hk, int hd, int S, float a_k, float a_v, int D, float* att, void* stream);
/* SwiGLU of one row (DeviceModel.forward llm/ref_model.py:246-250; ModelCompiler.ffn_up / silu_mul
 * llm/compile_model.py:295-328; expandFfn SahlExpandKernels.cpp:529): h1, h3 = the two W8A8 linears
 * of xq, u = F(F(h1 * RECIP(F(1 + EXP(F(h1 * -1))))) * h3) -> u_out[F] (required), then
 * hq, s_h = quant_act(u). */
int t2r_swiglu_w8a8(const int8_t* w1, const float* s_w1, const int8_t* w3, const float* s_w3, const int8_t* xq,
                    const float* s_x, int F, int K, float* u_out, int8_t* hq, float* s_h, void* stream);
/* MoE routing of rows scores[rows, E] (compiler/frontend/hf_generic.py:641-646;
 * compiler/tests/oracle.py:558-585): top-k ids in descending score order (equal scores: lower
 * id first), weights w = F(e * RECIP(red_sum(e))), e = EXP(F(v - v0)). E <= 64, k <= 8. */
int t2r_moe_route(const float* scores, int rows, int E, int k, int D, int32_t* ids, float* weights, void* stream);
/* The HF path's attention options at op level (compiler/frontend/hf_generic.py:153-187, 231-292):
 * t2r_attn_decode with flags T2R_ATTN_QSUM (qsum normalisation), ch_sk [Hk * hd] (K per channel:
 * q = F(q * ch_sk[c]) before its quant_act; NULL: per layer) and ch_av [Hk * hd] (V per channel: the
 * output channel scaled by ch_av[c] instead of a_v; NULL: per layer). */
#define T2R_ATTN_QSUM 1
int t2r_attn_decode_opt(const float* q, const int8_t* kc, const int8_t* vc, const int32_t* pos, int rows, int H,
                        int Hk, int hd, int S, float a_k, float a_v, int D, int flags, const float* ch_sk,
                        const float* ch_av, float* att, void* stream);
/* Prefill attention of M prompt rows q[M, H * hd] (already rotated, their KV rows already in the cache)
 * at positions pos[M], each row over the cache rows 0..pos[r] (the prompt chunk's attention:
 * expandAttnChunkBlocked, compiler/plugins/sa/transforms/SahlExpandKernels.cpp:1702; QModel.prefill's
 * per-row attention, compiler/frontend/qhf.py:356-409). Each row's result is t2r_attn_decode_opt's for
 * that row, bit for bit; rows run 16 at a time per query head on int8 MFMA where hd is a multiple of 16
 * (<= 128) and a row's scores fit in LDS, else row by row. Flags and per-channel scales as
 * t2r_attn_decode_opt. S = cache rows <= 8192. */
int t2r_attn_prefill(const float* q, const int8_t* kc, const int8_t* vc, const int32_t* pos, int M, int H, int Hk,
                     int hd, int S, float a_k, float a_v, int D, int flags, const float* ch_sk, const float* ch_av,
                     float* att, void* stream);
/* KV append with per-channel inverse scales inv_sk[kv_dim], inv_sv[kv_dim] (hf_generic.py:203-218):
 * kc[pos[r]][c] = to_i8(F(k[r][c] * inv_sk[c])); either vector may be NULL for the scalar one. */
int t2r_kv_append_ch(const float* k, const float* v, float inv_sk, float inv_sv, const float* inv_sk_ch,
                     const float* inv_sv_ch, int8_t* kc, int8_t* vc, const int32_t* pos, int rows, int kv_dim, int S,
                     void* stream);
/* The gated FFN up-projection of one row with the gate activation act: 0 SiLU (t2r_swiglu_w8a8),
 * 1 GELU-tanh (GeGLU: F(gelu(h1) * h3), gelu(x) = F(x * RECIP(F(EXP(z) + 1))),
 * z = F(x * F(A + F(F(x * x) * B))), A = f32(-2 sqrt(2/pi)), B = f32(A * 0.044715):
 * compiler/frontend/hf_generic.py:840-852), then hq, s_h = quant_act(u). */
int t2r_gated_ffn_w8a8(int act, const int8_t* w1, const float* s_w1, const int8_t* w3, const float* s_w3,
                       const int8_t* xq, const float* s_x, int F, int K, float* u_out, int8_t* hq, float* s_h,
                       void* stream);
/* First index of the largest value of each row (np.argmax; llm/ref_model.py:277). */
int t2r_argmax(const float* x, int rows, int n, int32_t* idx, void* stream);

/* ---------------------------------------------------------------- model level */
/* A decoder resident on the device. Pointers are device pointers except kv_consts (host).
 * Per-layer tensors are stacked with the layer first. */
typedef struct t2r_model_desc {
  int32_t abi_version;                 /* T2R_ABI_VERSION */
  int32_t dim, hidden, layers, heads, kv_heads, head_dim, vocab, seq_len;
  int32_t n_experts, top_k;            /* 0, 0: dense FFN */
  int32_t qk_norm, D;
  float eps;
  const int8_t* emb_q; const float* emb_s;          /* [vocab, dim], [vocab] */
  const int8_t* cls_q; const float* cls_s;          /* classifier (the embedding when tied) */
  const float* rms_att; const float* rms_ffn;       /* [L, dim] */
  const float* rms_final;                           /* [dim] */
  const float* q_norm; const float* k_norm;         /* [L, head_dim] (QK-norm) or NULL */
  const int8_t* wqkv; const float* s_wqkv;          /* [L, q + 2 kv, dim], [L, q + 2 kv] */
  const int8_t* wo; const float* s_wo;              /* [L, dim, q] */
  const int8_t* w1; const float* s_w1;              /* [L, hidden, dim] (dense) */
  const int8_t* w3; const float* s_w3;
  const int8_t* w2; const float* s_w2;              /* [L, dim, hidden] */
  const int8_t* router; const float* s_router;      /* [L, E, dim] (MoE) */
  const int8_t* wg; const float* s_wg;              /* [L, E, hidden, dim] */
  const int8_t* wu; const float* s_wu;
  const int8_t* wd; const float* s_wd;              /* [L, E, dim, hidden] */
  const float* rope_cos; const float* rope_sin;     /* [seq_len, head_dim / 2] */
  const float* kv_consts;                           /* HOST [L, 4]: 1/s_k, 1/s_v, a_k, a_v */
  int8_t* k_cache; int8_t* v_cache;                 /* [L, seq_len, kv_dim] */
  void* workspace; int64_t workspace_bytes;         /* see t2r_model_workspace_bytes */
  int32_t max_rows;                                 /* prefill rows per call the workspace holds */
  /* ABI 2: the numerics options of the reference's HF path (compiler/frontend/hf_generic.py), all
   * zero / NULL = DeviceModel's form. A descriptor with abi_version 1 ends before these fields and
   * is read with them off. */
  int32_t attn_qsum;        /* 1: qsum normalisation (:265-292): pq = to_i8(F(e * 127)), att =
                               F(F(f32(sum pq V) * F(RECIP(f32(sum pq)) * 127)) * a_v) */
  int32_t ffn_act;          /* FFN gate: 0 SiLU (SwiGLU), 1 GELU-tanh from EXP / RECIP (GeGLU, :840-852) */
  const float* kv_channel;  /* [L, 4, kv_dim] per cache channel: s_k, 1/s_k, 1/s_v, a_v (:153-187);
                               NULL when no layer has per-channel scales */
  const int32_t* kv_channel_flags;  /* HOST [L]: bit 0 K per channel (q = F(q * s_k) before its quant,
                                       kv_consts' a_k then f32(1 / sqrt(hd))), bit 1 V per channel; NULL: none */
} t2r_model_desc;

/* Bytes of workspace a model needs for prefill calls of up to max_rows rows (>= 1). */
int64_t t2r_model_workspace_bytes(const t2r_model_desc* desc, int max_rows);
/* Validates desc (shapes, pointers, workspace; layers <= 256) and returns a handle; copies desc. */
int t2r_model_create(const t2r_model_desc* desc, void** model);
/* No counterpart in the reference: for callers that cannot allocate device memory (serving loops that
 * forbid hipMalloc, code that later replays the model's calls from a captured HIP graph).
 * t2r_model_create with desc->workspace = NULL and desc->workspace_bytes = 0: the model's workspace is
 * the library's static device array of T2R_STATIC_WORKSPACE_BYTES on the current device, and the handle
 * comes from a fixed pool of 8, so the call allocates nothing. Creation itself clears the model's state
 * and synchronises the device: make the model before a capture starts; its decode, prefill and batched
 * calls are then capturable. Each handle keeps the state it carries from call to call (the status word,
 * the split attention's counters and sums) in its own part of the array (T2R_STATIC_STATE_BYTES in
 * all); the rest is one call's scratch, shared by all such models on the device: their calls must not
 * overlap, calls in sequence are fine. Returns T2R_ENOMEM when max_rows needs more than the array's
 * scratch part (T2R_STATIC_WORKSPACE_BYTES - T2R_STATIC_STATE_BYTES; t2r_model_workspace_bytes tells,
 * within the state's few KB), T2R_EINVAL when a workspace is given, T2R_ESTATE when the 8 handles are
 * taken. t2r_model_destroy returns the handle to the pool. */
#define T2R_STATIC_WORKSPACE_BYTES (16 * 1024 * 1024)
#define T2R_STATIC_STATE_BYTES (512 * 1024)
int t2r_model_create_static(const t2r_model_desc* desc, void** model);
void t2r_model_destroy(void* model);
/* One decode step (the reference's static token list: llm/compile_model.py:351-374, run per token
 * by llm/runtime.py:107-125): token and pos are read from DEVICE memory, so a captured HIP graph
 * replays unchanged (only the (pos, token) block changes, llm/compile_model.py:56-62). Writes the
 * logits [vocab] (may be NULL) and the greedy next token (may be NULL); the KV rows of pos are
 * written. flags: T2R_ADVANCE_POS increments *pos on the device after the step. */
#define T2R_ADVANCE_POS 1
int t2r_decode_step(void* model, const int32_t* token, int32_t* pos, float* logits, int32_t* next_token,
                    int flags, void* stream);
/* Prefill of M prompt rows tokens[M] at positions[M] (device arrays; each row a decode step at its
 * position: compiler/frontend/qhf.py:356-409): the KV rows are written, the logits of the last row
 * go to last_logits (may be NULL) and its greedy token to next_token (may be NULL).
 * M <= max_rows. Identical, bit for bit, to M decode steps. */
int t2r_prefill(void* model, const int32_t* tokens, const int32_t* positions, int M, float* last_logits,
                int32_t* next_token, void* stream);

/* t2r_prefill at the positions start .. start + M - 1 (the reference's chunk schedule,
 * compiler/frontend/export.py:69-72, compiler/runtime/tools/sa_llm_run.c:255-330). Every row then
 * attends to at most start + M positions, which sizes the attention's score rows (and lets more
 * of its workgroups share a CU than the cache length would); results are those of t2r_prefill.
 * 0 <= start, start + M <= seq_len, M <= max_rows. */
int t2r_prefill_at(void* model, const int32_t* tokens, int start, int M, float* last_logits, int32_t* next_token,
                   void* stream);

/* Batched decode: one token of each of B sequences (BatchLlamaDevice.step llm/runtime.py:193-208;
 * compile_batch.BatchCompiler llm/compile_batch.py:1-25): row b is sequence b at positions[b] with
 * tokens[b], its KV cache at k_caches / v_caches + b * cache_stride bytes (each laid out as the
 * model's k_cache / v_cache: [layers, seq_len, kv_dim] int8; cache_stride >= that size when B > 1).
 * The linear layers run once over the B rows (int8 MFMA), attention per row; logits [B, vocab]
 * fp32, next_tokens [B] the first maximum per row (may be NULL). Row b is bit-identical to a decode
 * step of sequence b alone. B <= max_rows. The model's own caches are not touched. */
int t2r_decode_batch(void* model, const int32_t* tokens, const int32_t* positions, int B, int8_t* k_caches,
                     int8_t* v_caches, int64_t cache_stride, float* logits, int32_t* next_tokens, void* stream);

/* The model's status word (the reference's per-list status, llm/runtime.py:116-119): bit 0 a token
 * outside [0, vocab) was embedded (row 0 read instead); bit 1 a bounded wait between the workgroups of
 * a head's decode attention ran out (its output is then not to be trusted); bit 2 a row's position
 * (device memory: a replayed graph's advancing position, say) was outside the cache, and its attention
 * read no cache row and wrote nothing (no cache row, no output). The bits stay set until cleared. Waits for the device; clear != 0
 * then zeroes the word. */
int t2r_model_status(void* model, int32_t* out, int clear);

/* Kernel timing of a resident model with HIP events on the launch stream (the GPU counterpart of
 * the reference's event counters and per-list cycle counts: rtl/sysarray/sa_perf.v,
 * driver/pynq_matmul.py:969-981, 1029-1066). t2r_model_profile creates 2 * max_launches events
 * (set-up time, not the hot path) and, for the kernel classes in mask (1 << T2R_PROF_*), records
 * one event before and one after every launch of later decode / prefill calls, until the pool is
 * full; mask 0 frees the pool. t2r_model_profile_read waits for the recorded events and returns
 * the number of launches recorded (kinds[i], ms[i] for the first max of them), then empties the
 * record. Returns a negative code on error. */
enum {
  T2R_PROF_QKV = 0,        /* RMSNorm + quant + Wqkv GEMV                        */
  T2R_PROF_ATTN = 1,       /* QK-norm, RoPE, KV append, attention                */
  T2R_PROF_WO = 2,         /* quant + Wo GEMV + residual                         */
  T2R_PROF_FFN_UP = 3,     /* RMSNorm + quant + W1 / W3 GEMV + SiLU gate (MoE: expert gate / up) */
  T2R_PROF_FFN_DOWN = 4,   /* quant + W2 GEMV + residual (MoE: expert down + combine) */
  T2R_PROF_CLS = 5,        /* final RMSNorm + quant + classifier GEMV + argmax   */
  T2R_PROF_ROUTE = 6,      /* MoE router + top-k                                 */
  T2R_PROF_OTHER = 7       /* embedding, step end                                */
};
int t2r_model_profile(void* model, int mask, int max_launches);
int t2r_model_profile_read(void* model, int32_t* kinds, float* ms, int max);

#ifdef __cplusplus
}
#endif
#endif /* T2R_H */
