/*
 * include/apus_hip.h -- C ABI of libapus_hip.so, the MI355X (gfx950)
 * implementation of the apus-qwen attention hot path: the Gated DeltaNet
 * ops (reference c/gdn.h) and the gated-GQA ops (reference c/attn.h).
 *
 * Plain C: no HIP or torch types. bf16 travels as uint16_t codes, fp32 as
 * float, dims as size_t, exactly as in the reference headers. Every entry
 * point returns int: 0 when it handled the op, nonzero otherwise (the
 * reference hook convention, c/backend_metal.h:16-20 and c/bf16.h:199-205:
 * a nonzero return means "run your CPU kernel"); apus_hip_last_error()
 * gives the message. Setting APUS_HIP_DISABLE=1 in the environment makes
 * every entry point return APUS_HIP_ERR_DISABLED, which forces a host
 * engine onto its CPU path (the forced-fallback switch of
 * c/backend_metal.mm:490-495).
 *
 * The library is driven by one compute thread, like the reference engine
 * (c/pool.h:7-16); it is not safe for concurrent callers.
 *
 * Tier 1 (drop-in): name-for-name replacements of the reference ops with
 *   the same argument lists, HOST pointers, synchronous. Results equal
 *   the reference scalar anchors up to libm ulps (expf/log1pf in the
 *   gates); see each declaration for the reference signature replaced.
 * Tier 2 (batched, device-resident): DEVICE pointers, stream-ordered on
 *   the library's current stream (apus_hip_set_stream), state and caches
 *   kept in HBM across calls.
 */
#ifndef APUS_HIP_H
#define APUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define APUS_HIP_OK 0
#define APUS_HIP_ERR_UNSUPPORTED 1
#define APUS_HIP_ERR_DISABLED 2
#define APUS_HIP_ERR_ARGUMENT 3
#define APUS_HIP_ERR_HIP 4

/* ---- library control ------------------------------------------------
 * apus_hip_init mirrors `int apus_metal_enable(char *err, size_t errcap)`
 * (c/bf16.h:250-254): 0 on success, else nonzero with a message in err.
 * Calling it is optional; the first op initialises device 0. */
int    apus_hip_init(int device, char *err, size_t errcap);
/* mirrors apus_metal_is_enabled (c/bf16.h:256) */
int    apus_hip_is_enabled(void);
size_t apus_hip_last_error(char *buf, size_t cap);
/* stream is a hipStream_t passed as void* (NULL = the null stream) */
int    apus_hip_set_stream(void *stream);
int    apus_hip_synchronize(void);
/* Bounded device waits (no counterpart in the reference, whose ops run on
 * one host thread): a kernel whose wavefronts wait on each other (the
 * decode score ring) gives up after `polls` polls, marks the call failed
 * and exits normally; apus_hip_synchronize then returns APUS_HIP_ERR_HIP
 * naming the kernel. 0 restores the default (2^22 polls, about a quarter
 * of a second). A tiny limit exists to test the error path. */
int    apus_hip_set_spin_limit(uint32_t polls);
/* Host-only check of the decode split plan (no device needed; no
 * counterpart in the reference): for B sequences of 1..4 new tokens after
 * pos0[s] cached, nkv kv heads and `cus` compute units, walks the runs the
 * decode kernels would be given and fills out[12] (see attn_mixer.hip):
 * out[1] counts runs whose two group enumerations of the score ring
 * disagree, out[4]/out[9] keys missed or covered twice, out[5]/out[10]
 * slot collisions, out[6]/out[11] mismatched pair run ranges -- all zero
 * for a sound plan. */
int    apus_hip_attn_split_check(size_t B, const int32_t *cu, const int32_t *pos0,
                                 size_t nkv, size_t cus, int64_t *out);
/* Device memory for hosts that do not link HIP themselves (state, KV). */
int    apus_hip_malloc(void **dptr, size_t bytes);
int    apus_hip_free(void *dptr);
int    apus_hip_memcpy_h2d(void *dst, const void *src, size_t bytes);
int    apus_hip_memcpy_d2h(void *dst, const void *src, size_t bytes);
int    apus_hip_memset(void *dst, int value, size_t bytes);
/* Per-kernel timing (no counterpart in the reference; for benchmarks and
 * profiling hosts). enable(1) clears and starts recording a pair of
 * events on the library stream around every mixer kernel launch;
 * enable(0) stops. get() synchronizes the stream and returns the summed
 * milliseconds and launch count recorded for one kernel name (e.g.
 * "k_gdn_chunk_scan"). */
int    apus_hip_timing_enable(int on);
int    apus_hip_timing_get(const char *kernel, double *total_ms, size_t *count);

/* Named-intermediate capture, the hot-path fields of the reference's
 * ApusLayerTrace (c/layer.h:172-189; filled per token at c/layer.h:275-285
 * and 324-330). While a trace is set, every tier-2 GDN mixer call
 * (apus_hip_gdn_decode, _decode_into, _decode_slots, _prefill,
 * _prefill_slots) writes, for each of its packed tokens t:
 *   qkv_conv [t][conv_dim] bf16  conv1d+SiLU output (q|k|v)
 *   beta     [t][hv]       bf16  sigmoid(b)
 *   gdecay   [t][hv]       f32   the decay g
 *   rec_o    [t][hv*dv]    bf16  rnd(o) of the recurrence
 *   onorm    [t][hv*dv]    bf16  the gated RMSNorm output (= the mixer's y)
 * and every tier-2 attention call (decode, prefill, paged or flat):
 *   qf       [t][nh*d]     bf16  q after (1+w) RMSNorm and RoPE
 *   kf       [t][nkv*d]    bf16  k after norm and RoPE (the appended row)
 *   attno    [t][nh*d]     bf16  the attention output before the gate
 *   mgate    [t][nh*d]     bf16  rnd(sigmoid(gate))
 * DEVICE pointers; any member may be NULL; NULL structs stop tracing. The
 * values are those the kernels compute (the chunked prefill's rec_o is its
 * tolerance class). Tracing adds work and is meant for checking, as the
 * reference uses its trace for the stage gates (tests/m4c). */
typedef struct {
    uint16_t *qkv_conv, *beta;
    float    *gdecay;
    uint16_t *rec_o, *onorm;
} ApusHipGdnTrace;
typedef struct {
    uint16_t *qf, *kf, *attno, *mgate;
} ApusHipAttnTrace;
int apus_hip_trace_set(const ApusHipGdnTrace *gdn, const ApusHipAttnTrace *attn);

/* ---- Tier 1: GDN ops (c/gdn.h) -------------------------------------- */
/* replaces apus_gdn_conv1d      (c/gdn.h:107-108, impl 314-318) */
int apus_hip_gdn_conv1d(const uint16_t *x, const uint16_t *w, uint16_t *out,
                        size_t C, size_t T, uint16_t *state);
/* replaces apus_gdn_conv1d_step (c/gdn.h:111-112, impl 305-312) */
int apus_hip_gdn_conv1d_step(const uint16_t *x, const uint16_t *w,
                             uint16_t *out, size_t C, uint16_t *state);
/* replaces apus_gdn_decay       (c/gdn.h:123-124, impl 322-363) */
int apus_hip_gdn_decay(const uint16_t *a, const float *A_log,
                       const float *dt_bias, float *g, size_t H);
/* replaces apus_gdn_beta        (c/gdn.h:133, impl 366-399) */
int apus_hip_gdn_beta(const uint16_t *b, uint16_t *beta, size_t H);
/* replaces apus_gdn_l2norm      (c/gdn.h:141-142, impl 402-465) */
int apus_hip_gdn_l2norm(const uint16_t *x, float *y, size_t H, size_t D,
                        float scale);
/* replaces apus_gdn_step        (c/gdn.h:153-156, impl 587-595) */
int apus_hip_gdn_step(float *S, const float *q, const float *k,
                      const uint16_t *v, const float *g, const uint16_t *beta,
                      float *o, size_t H, size_t Dk, size_t Dv);
/* replaces apus_gdn_step_mt     (c/gdn.h:159-162, impl 619-625) */
int apus_hip_gdn_step_mt(float *S, const float *q, const float *k,
                         const uint16_t *v, const float *g,
                         const uint16_t *beta, float *o, size_t H, size_t Dk,
                         size_t Dv);
/* replaces apus_gdn_recurrent   (c/gdn.h:166-169, impl 627-635) */
int apus_hip_gdn_recurrent(float *S, const float *q, const float *k,
                           const uint16_t *v, const float *g,
                           const uint16_t *beta, float *o, size_t T,
                           size_t H, size_t Dk, size_t Dv);
/* replaces apus_gdn_onorm       (c/gdn.h:183-184, impl 639-661) */
int apus_hip_gdn_onorm(const uint16_t *o, const uint16_t *z,
                       const uint16_t *w, uint16_t *y, size_t H, size_t D);

/* ---- Tier 1: attention ops (c/attn.h) ------------------------------- */
/* replaces apus_attn_rmsnorm    (c/attn.h:87-88, impl 175-186) */
int apus_hip_attn_rmsnorm(const uint16_t *x, const uint16_t *w, uint16_t *y,
                          size_t N);
/* replaces apus_attn_rope       (c/attn.h:99-100, impl 244-266) */
int apus_hip_attn_rope(const uint16_t *x, uint16_t *y, size_t D, size_t rot,
                       float pos, double theta);
/* replaces apus_attn_gqa        (c/attn.h:112-115, impl 450-464);
 * abuf/ebuf are accepted and unused (device scratch is used instead) */
int apus_hip_attn_gqa(const uint16_t *q, const uint16_t *kc,
                      const uint16_t *vc, uint16_t *o, size_t Tq, size_t Tk,
                      size_t H, size_t Hkv, size_t D, float scale,
                      uint16_t *abuf, float *ebuf);
/* replaces apus_attn_gqa_decode (c/attn.h:119-122, impl 466-471) */
int apus_hip_attn_gqa_decode(const uint16_t *q, const uint16_t *kc,
                             const uint16_t *vc, uint16_t *o, size_t Tk,
                             size_t H, size_t Hkv, size_t D, float scale,
                             uint16_t *abuf, float *ebuf);
/* replaces apus_attn_gqa_mt     (c/attn.h:128-131, impl 507-513) */
int apus_hip_attn_gqa_mt(const uint16_t *q, const uint16_t *kc,
                         const uint16_t *vc, uint16_t *o, size_t Tq,
                         size_t Tk, size_t H, size_t Hkv, size_t D,
                         float scale);
/* replaces apus_attn_gqa_decode_mt (c/attn.h:132-135, impl 515-520) */
int apus_hip_attn_gqa_decode_mt(const uint16_t *q, const uint16_t *kc,
                                const uint16_t *vc, uint16_t *o, size_t Tk,
                                size_t H, size_t Hkv, size_t D, float scale);
/* replaces apus_attn_outgate    (c/attn.h:151-152, impl 524-531) */
int apus_hip_attn_outgate(const uint16_t *o, const uint16_t *gate,
                          uint16_t *y, size_t N);

/* ---- Tier 2: batched device-resident mixers ---------------------------
 * A "mixer" is the hot path between a layer's input projections and its
 * output projection, i.e. the op sequence of c/layer.h:250-273 (GDN) and
 * c/layer.h:300-322 (full attention), for B independent sequences.
 * Tokens are packed: sequence s owns rows cu[s] .. cu[s+1]-1 (cu is a
 * HOST array of B+1 ascending offsets, cu[0] = 0). Weight, activation,
 * state and cache pointers are DEVICE pointers. */

/* GDN layer weights + dims (the hot fields of ApusLayerCfg/ApusLayerW,
 * c/layer.h:113-157). Device pointers. */
typedef struct {
    size_t hk, hv, dk, dv;          /* 16, 32, 128, 128 */
    const uint16_t *conv_w;         /* [conv_dim, 4] bf16 */
    const float *A_log, *dt_bias;   /* [hv] f32 */
    const uint16_t *onorm_w;        /* [dv] bf16, direct weight */
} ApusHipGdnLayer;

/* Device state layout. Tier-2 GDN calls keep each (sequence, v-head)
 * recurrent state -- reference layout S[i][j], i < dk, j < dv, fp32
 * (c/gdn.h:149-156) -- "column packed" in HBM: element S[i][j] of a
 * 128x128 matrix sits at float offset ((j/64*32 + i/4)*64 + j%64)*4 + i%4.
 * A wavefront owning 64 value columns then streams its tile with 16-byte
 * loads. These convert nmat consecutive matrices between the reference
 * layout and the device layout (device pointers, no aliasing). */
int apus_hip_gdn_state_pack(const float *S_ref, float *S_dev, size_t nmat);
int apus_hip_gdn_state_unpack(const float *S_dev, float *S_ref, size_t nmat);

/* Fused GDN decode / verify: for each sequence, its tokens in order run
 * conv1d+SiLU, beta, decay, l2norm, the delta-rule step and the gated
 * RMSNorm (c/layer.h:250-273 per token; 1..k tokens per sequence, the MTP
 * verify shape of c/mtp.h:36-75).
 *   qkv [Ttot, 2*hk*dk + hv*dv], z [Ttot, hv*dv], a,b [Ttot, hv] bf16;
 *   conv_state [B, conv_dim*3] bf16 (in/out); S [B, hv] matrices of
 *   dk x dv f32 in the device layout above (in/out); y [Ttot, hv*dv] bf16
 *   (feeds w_out). y and S equal the reference anchors up to libm ulps.
 * Supports dk = dv = 128 and hv = 2*hk (the model's shape). */
int apus_hip_gdn_decode(const ApusHipGdnLayer *L, size_t B,
                        const int32_t *cu, const uint16_t *qkv,
                        const uint16_t *z, const uint16_t *a,
                        const uint16_t *b, uint16_t *conv_state, float *S,
                        uint16_t *y);

/* GDN decode / verify out of place: as apus_hip_gdn_decode, reading each
 * sequence's conv state and S from conv_in / S_in and writing the updated
 * ones to conv_out / S_out (the same buffers, or disjoint ones). A sequence
 * with no tokens in cu is skipped and its output state left untouched.
 * This is the device form of the MTP snapshot/rollback of c/mtp.h:36-75
 * (snapshot S and conv state, verify, on a partial reject restore the
 * snapshot and re-feed the accepted prefix): with the input set kept as the
 * snapshot, a verify writes the output set, and a rollback re-feeds the
 * accepted prefix of the rejected sequences from the same input set into
 * the output set; no state is copied. Full-attention layers roll back by
 * their position alone (pos0 of the next call; rows past it are never
 * read, c/mtp.h:64-68). */
int apus_hip_gdn_decode_into(const ApusHipGdnLayer *L, size_t B,
                             const int32_t *cu, const uint16_t *qkv,
                             const uint16_t *z, const uint16_t *a,
                             const uint16_t *b, const uint16_t *conv_in,
                             const float *S_in, uint16_t *conv_out,
                             float *S_out, uint16_t *y);

/* GDN decode / verify on a state pool (no counterpart in the reference,
 * whose layer state is one sequence's, c/layer.h:159-167): conv and S are
 * the base of a layer's slot arrays -- slot i at conv + i*conv_dim*3 and
 * S + i*hv*dk*dv (device layout) -- and sequence s reads its state from
 * slot_in[s] and writes it to slot_out[s] (HOST arrays). slot_out[s] ==
 * slot_in[s] decodes in place; a different output slot keeps the input as
 * an MTP snapshot (the rollback of c/mtp.h:70-75 is then a re-feed from the
 * kept slot). The output slots of sequences with tokens must be distinct
 * and none may be another sequence's input slot. */
int apus_hip_gdn_decode_slots(const ApusHipGdnLayer *L, size_t B,
                              const int32_t *slot_in, const int32_t *slot_out,
                              const int32_t *cu, const uint16_t *qkv,
                              const uint16_t *z, const uint16_t *a,
                              const uint16_t *b, uint16_t *conv, float *S,
                              uint16_t *y);

/* Chunked GDN prefill: the same layer and arguments as apus_hip_gdn_decode
 * for sequences of any length (c/layer.h:427-492, the prompt path; the
 * reference steps the recurrence token by token, c/gdn.h:627-635). The
 * recurrence runs in chunks of 64 tokens in the WY/UT form on the bf16
 * MFMA with fp32 accumulation, every fp32 operand split into hi/lo bf16
 * parts (q and k enter as their exact bf16 conv codes): conv_state and the
 * token-parallel ops equal the reference anchors up to libm ulps; S and y
 * are a tolerance class of the sequential recurrence (state within 1e-4
 * relative, y within bf16 rounding of the sequential result). Library
 * scratch grows with the token count: about 96 KiB per (chunk of 64
 * tokens, v-head) plus 8 KiB per token. */
int apus_hip_gdn_prefill(const ApusHipGdnLayer *L, size_t B,
                         const int32_t *cu, const uint16_t *qkv,
                         const uint16_t *z, const uint16_t *a,
                         const uint16_t *b, uint16_t *conv_state, float *S,
                         uint16_t *y);

/* apus_hip_gdn_prefill that allocates nothing (no counterpart in the
 * reference; for callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, hosts that forbid hipMalloc).
 * Same arguments, results bit-identical to apus_hip_gdn_prefill. The
 * intermediates live in one fixed per-device scratch array of 96 MiB,
 * reserved when the library initialises a device and held until the
 * process ends: a call needs about 8 KiB per token plus 3.0 MiB per
 * (sequence, chunk of 64 tokens), so one sequence of up to ~1700 tokens
 * (longer prompts are prefilled in successive calls: the state carries
 * over); at most 400 sequences and no slot map. A larger call returns
 * APUS_HIP_ERR_UNSUPPORTED with the size it needs; so does a call made
 * while a GDN trace is set (capturing it would allocate). Calls on one GPU share
 * that GPU's scratch: calls that overlap (two streams) race. */
int apus_hip_gdn_prefill_noalloc(const ApusHipGdnLayer *L, size_t B,
                                 const int32_t *cu, const uint16_t *qkv,
                                 const uint16_t *z, const uint16_t *a,
                                 const uint16_t *b, uint16_t *conv_state,
                                 float *S, uint16_t *y);

/* apus_hip_gdn_prefill on a state pool: sequence s's state is slot
 * slots[s] (HOST array, distinct for sequences with tokens) of the slot
 * arrays conv / S (layout as apus_hip_gdn_decode_slots). */
int apus_hip_gdn_prefill_slots(const ApusHipGdnLayer *L, size_t B,
                               const int32_t *slots, const int32_t *cu,
                               const uint16_t *qkv, const uint16_t *z,
                               const uint16_t *a, const uint16_t *b,
                               uint16_t *conv, float *S, uint16_t *y);

/* Full-attention layer weights + dims (hot fields of ApusLayerCfg/W,
 * c/layer.h:113-157). Device pointers. */
typedef struct {
    size_t nh, nkv, d, rot;         /* 16, 2, 256, 64 */
    double theta;                   /* 1e7 */
    const uint16_t *qn_w, *kn_w;    /* [d] bf16, (1+w) storage */
} ApusHipAttnLayer;

/* Device KV-cache layout: blocks of 32 positions. Block b (positions
 * 32b .. 32b+31) of a sequence is a K block [nkv][32][d] (d contiguous) and
 * a V block [nkv][d][32] (transposed), bf16, at block id `id`:
 *   K: kcache + id * nkv*32*d,   V: vcache + id * nkv*d*32.
 * Flat caches (apus_hip_attn_decode / _prefill): sequence s of the batch
 * owns ids s*(max_seq/32) .. s*(max_seq/32) + max_seq/32 - 1 in order,
 * i.e. max_seq*nkv*d elements of each array, max_seq a multiple of 32.
 * Paged caches (ApusHipKvCache below): ids come from a block table. The
 * reference keeps both as [max_seq][nkv][d] (c/layer.h:164-165); pack /
 * unpack convert the first ntok positions of one sequence (device
 * pointers). */
int apus_hip_attn_cache_pack(const uint16_t *kc_ref, const uint16_t *vc_ref,
                             size_t ntok, size_t nkv, size_t d,
                             uint16_t *kcache, uint16_t *vcache, size_t max_seq);
int apus_hip_attn_cache_unpack(const uint16_t *kcache, const uint16_t *vcache,
                               size_t ntok, size_t nkv, size_t d, size_t max_seq,
                               uint16_t *kc_ref, uint16_t *vc_ref);

/* Paged KV cache (no counterpart in the reference, whose cache is one
 * flat [max_seq][nkv][d] array per sequence, c/model.h:615-616): block
 * arrays k and v (device) and a device block table [rows][max_blocks] whose
 * entry [h][b] is the id of block b of the sequence at table row h. The
 * *_paged calls take, per sequence of the batch, its table row (HOST array
 * rows[B]); a sequence may use blocks 0 .. ceil((pos0+new)/32) - 1 of its
 * row. apus_hip_kv_pool_* below manage such a cache. The table has
 * max_rows rows; a call naming a row >= max_rows is refused. row_blocks
 * (HOST array [max_rows], nullable) holds the blocks each row has
 * reserved (-1: row closed); when set, a call whose new tokens reach past
 * a row's reserved blocks is refused instead of writing through stale
 * table entries. apus_hip_kv_pool_cache fills both. */
typedef struct {
    uint16_t *k, *v;
    const int32_t *block_table;
    size_t max_blocks;
    size_t max_rows;
    const int32_t *row_blocks;
} ApusHipKvCache;
int apus_hip_attn_cache_pack_paged(const uint16_t *kc_ref, const uint16_t *vc_ref,
                                   size_t ntok, size_t nkv, size_t d,
                                   const ApusHipKvCache *kv, int32_t row);
int apus_hip_attn_cache_unpack_paged(const ApusHipKvCache *kv, int32_t row,
                                     size_t ntok, size_t nkv, size_t d,
                                     uint16_t *kc_ref, uint16_t *vc_ref);

/* Full-attention causal prefill for B sequences of any length (c/layer.h:
 * 498-564: per token q/k (1+w) RMSNorm, partial RoPE, cache append, then
 * causal GQA of every new token over the cache, sigmoid output gate).
 * Arguments as apus_hip_attn_decode with no limit on new tokens per
 * sequence (pos0[s] + new tokens <= max_seq). The attention runs as an
 * MFMA flash-attention kernel; y is a tolerance class of the reference
 * (|c - r| <= 2e-3 (|r| + sum_j |P_j V_j|)). Supports d=256, rot=64,
 * nh=8*nkv. */
int apus_hip_attn_prefill(const ApusHipAttnLayer *L, size_t B,
                          const int32_t *cu, const int32_t *pos0,
                          const uint16_t *qg, const uint16_t *k,
                          const uint16_t *v, uint16_t *kcache,
                          uint16_t *vcache, size_t max_seq, uint16_t *y);

/* Full-attention decode / verify for B sequences (c/layer.h:300-322 per
 * token: q/k (1+w) RMSNorm, partial RoPE at each token's position, cache
 * append, causal GQA over the cache, sigmoid output gate). Sequence s has
 * pos0[s] tokens cached (HOST array) and cu[s+1]-cu[s] in 1..4 new tokens;
 * new token t sits at position pos0[s]+t and attends keys 0..pos0[s]+t.
 *   qg [Ttot, nh, 2d] ([q|gate] per head), k, v [Ttot, nkv, d] bf16;
 *   y [Ttot, nh*d] bf16 (feeds wo).
 * Split-K over the context on MFMA. Supports d=256, rot=64, nh=8*nkv. */
int apus_hip_attn_decode(const ApusHipAttnLayer *L, size_t B,
                         const int32_t *cu, const int32_t *pos0,
                         const uint16_t *qg, const uint16_t *k,
                         const uint16_t *v, uint16_t *kcache,
                         uint16_t *vcache, size_t max_seq, uint16_t *y);

/* apus_hip_attn_prefill / _decode on a paged cache: sequence s of the
 * batch lives at block-table row rows[s] (HOST array). */
int apus_hip_attn_prefill_paged(const ApusHipAttnLayer *L, size_t B,
                                const int32_t *rows, const int32_t *cu,
                                const int32_t *pos0, const uint16_t *qg,
                                const uint16_t *k, const uint16_t *v,
                                const ApusHipKvCache *kv, uint16_t *y);
int apus_hip_attn_decode_paged(const ApusHipAttnLayer *L, size_t B,
                               const int32_t *rows, const int32_t *cu,
                               const int32_t *pos0, const uint16_t *qg,
                               const uint16_t *k, const uint16_t *v,
                               const ApusHipKvCache *kv, uint16_t *y);

/* ---- state managers (no counterpart in the reference; its engine keeps
 * one sequence's state per layer, c/model.h:615-616) ----------------------
 * KV pool: nlayers full-attention layers' block arrays of nblocks blocks
 * each (32 positions x nkv x d, K and V) sharing one block table of
 * max_rows rows x max_blocks entries. A sequence opens a row, reserves
 * positions as it grows (blocks are taken from a free list; the table
 * update is stream-ordered on the library stream) and closes the row when
 * it ends; a rollback is a position rewind (pos0 of the next call), with
 * no table change. apus_hip_kv_pool_cache gives layer l's ApusHipKvCache
 * for the *_paged calls. Close a row only after the work that reads it has
 * been enqueued before the next reserve of its blocks by another row (the
 * library stream orders them). */
typedef struct ApusHipKvPool ApusHipKvPool;
int apus_hip_kv_pool_create(size_t nlayers, size_t nkv, size_t d, size_t nblocks,
                            size_t max_rows, size_t max_blocks, ApusHipKvPool **out);
int apus_hip_kv_pool_destroy(ApusHipKvPool *pool);
int apus_hip_kv_pool_cache(const ApusHipKvPool *pool, size_t layer,
                           ApusHipKvCache *out);
int apus_hip_kv_seq_open(ApusHipKvPool *pool, int32_t *row);
int apus_hip_kv_seq_reserve(ApusHipKvPool *pool, int32_t row, size_t ntok);
int apus_hip_kv_seq_close(ApusHipKvPool *pool, int32_t row);
size_t apus_hip_kv_pool_free_blocks(const ApusHipKvPool *pool);

/* GDN state pool: nlayers GDN layers' slot arrays of nslots sequence
 * states each (conv state + recurrent state); apus_hip_gdn_pool_state
 * gives layer l's bases for the *_slots calls. A slot opened for a new
 * sequence starts from zero state in every layer (c/layer.h:219-227,
 * stream-ordered). */
typedef struct ApusHipGdnPool ApusHipGdnPool;
int apus_hip_gdn_pool_create(size_t nlayers, size_t hk, size_t hv, size_t dk,
                             size_t dv, size_t nslots, ApusHipGdnPool **out);
int apus_hip_gdn_pool_destroy(ApusHipGdnPool *pool);
int apus_hip_gdn_pool_state(const ApusHipGdnPool *pool, size_t layer,
                            uint16_t **conv, float **S);
int apus_hip_gdn_slot_open(ApusHipGdnPool *pool, int32_t *slot);
int apus_hip_gdn_slot_close(ApusHipGdnPool *pool, int32_t slot);
/* Copy one sequence's state of one layer between an open slot and arrays
 * in the reference layout (conv [conv_dim*3] bf16, S [hv][dk][dv] f32,
 * c/layer.h:159-162; DEVICE pointers): load imports a state (a snapshot,
 * or one computed elsewhere), store exports it. Stream-ordered. */
int apus_hip_gdn_slot_load(ApusHipGdnPool *pool, size_t layer, int32_t slot,
                           const uint16_t *conv, const float *S);
int apus_hip_gdn_slot_store(ApusHipGdnPool *pool, size_t layer, int32_t slot,
                            uint16_t *conv, float *S);

/* ---- weight container reader (replaces c/st.h:64-89: apus_st_open /
 * apus_st_find / apus_st_set_open / apus_st_set_get) -----------------------
 * A path is one .safetensors shard or a directory holding
 * model.safetensors.index.json and its shards. Shards are opened header-
 * only; apus_hip_st_read copies one tensor's payload (pread) into caller
 * memory. Host-side only: these calls need no device and ignore
 * APUS_HIP_DISABLE. Codes of ApusHipStTensor.dtype follow the reference's
 * ApusStDtype order (c/st.h:44-48). */
#define APUS_HIP_ST_I8 0
#define APUS_HIP_ST_U8 1
#define APUS_HIP_ST_F8_E8M0 2
#define APUS_HIP_ST_F8_E4M3 3
#define APUS_HIP_ST_BF16 4
#define APUS_HIP_ST_F16 5
#define APUS_HIP_ST_F32 6
#define APUS_HIP_ST_I32 7
#define APUS_HIP_ST_I64 8
#define APUS_HIP_ST_OTHER 9
#define APUS_HIP_ST_MAX_NDIM 8
typedef struct {
    char    name[160];
    int     dtype;
    int     ndim;
    int64_t shape[APUS_HIP_ST_MAX_NDIM];
    size_t  nbytes;
} ApusHipStTensor;
typedef struct ApusHipSt ApusHipSt;
int    apus_hip_st_open(const char *path, ApusHipSt **out);
int    apus_hip_st_close(ApusHipSt *st);
size_t apus_hip_st_ntensors(const ApusHipSt *st);
int    apus_hip_st_find(ApusHipSt *st, const char *name, ApusHipStTensor *info);
int    apus_hip_st_read(ApusHipSt *st, const char *name, void *dst, size_t cap);

/* One layer's hot-path weights from a container onto the device, under the
 * reference's tensor names (c/model.h:440-490): GDN layer L reads
 * model.language_model.layers.L.linear_attn.{conv1d.weight, norm.weight}
 * (BF16) and .{A_log, dt_bias} (F32, or BF16 widened as c/model.h:249-275
 * does); a full-attention layer reads .self_attn.{q_norm,k_norm}.weight
 * (BF16). The device copies belong to the layer struct until *_free. */
int apus_hip_gdn_layer_load(ApusHipSt *st, int layer, size_t hk, size_t hv,
                            size_t dk, size_t dv, ApusHipGdnLayer *out);
int apus_hip_attn_layer_load(ApusHipSt *st, int layer, size_t nh, size_t nkv,
                             size_t d, size_t rot, double theta,
                             ApusHipAttnLayer *out);
int apus_hip_gdn_layer_free(ApusHipGdnLayer *layer);
int apus_hip_attn_layer_free(ApusHipAttnLayer *layer);

/* ---- projections on either side of the path (c/bf16.h:178-231) --------
 * y[m][o] = rnd(sum_k w[o][k] * x[m][k]), w [O][K], x [M][K], y [M][O],
 * bf16 codes, fp32 accumulation. */

/* Drop-ins for the reference's backend hook slots bf16_gemv / bf16_gemm
 * (ApusBackendHooks, c/backend_metal.h:68-75, called from
 * apus_bf16_gemv_hot / apus_bf16_gemm_hot, c/bf16.h:199-231) with their
 * argument lists. HOST pointers. The k sum runs in the reference's order
 * (ascending k, one rounding per multiply and per add, c/bf16.h:285-293),
 * so y is bitwise the reference's. (The multiply and add run fused: a
 * product of two bf16 values is exact in fp32, so the fused form rounds
 * where the reference does; only a product below 2^-126 in magnitude,
 * while the running sum is that small too, could round differently.) w must be a stable weight: its device
 * copy is made at the first call and reused while (w, O*K) is unchanged
 * (the Metal backend's stable-pointer rule, c/backend_metal.h:42-48);
 * apus_hip_bf16_weights_release drops every copy. */
int apus_hip_bf16_gemv(const uint16_t *w, const uint16_t *x, uint16_t *y,
                       size_t O, size_t K);
int apus_hip_bf16_gemm(const uint16_t *w, const uint16_t *x, uint16_t *y,
                       size_t M, size_t O, size_t K);
int apus_hip_bf16_weights_release(void);

/* Device-pointer forms (no counterpart in the reference; the tier-2 calls
 * around the device-resident mixers). _dev: the reference's order, bitwise,
 * one lane per output (decode-sized M). _mfma_dev: a hand-written
 * 32x32x16 bf16 MFMA GEMM with fp32 accumulation for any M (tile shape
 * chosen per call shape; K % 32 == 0, 16-byte aligned w and x, else
 * APUS_HIP_ERR_UNSUPPORTED); it sums in its own order, a tolerance class of
 * the reference (|c - r| <= 2e-3 (|r| + sum_k |w x|)), and its result does
 * not depend on the tile shape (every element accumulates its k16 steps
 * in order). */
int apus_hip_bf16_gemm_dev(const uint16_t *w, const uint16_t *x, uint16_t *y,
                           size_t M, size_t O, size_t K);
int apus_hip_bf16_gemm_mfma_dev(const uint16_t *w, const uint16_t *x,
                                uint16_t *y, size_t M, size_t O, size_t K);

/* ---- one layer's mixer with its projections (c/layer.h:236-331) --------
 * The reference's per-token layer body around the mixer: the input
 * projections of the normed input ln1, the mixer, the output projection.
 * Device pointers; the weights keep the reference's layouts
 * (ApusLayerW, c/layer.h:133-157), [rows][hidden] bf16, 16-byte aligned. */
typedef struct {
    size_t hidden;                  /* H = 2048 */
    const uint16_t *w_qkv;          /* [conv_dim][H] */
    const uint16_t *w_z;            /* [value_dim][H] */
    const uint16_t *w_b, *w_a;      /* [hv][H] */
    const uint16_t *w_out;          /* [H][value_dim] */
} ApusHipGdnProj;
typedef struct {
    size_t hidden;                  /* H = 2048 */
    const uint16_t *wq;             /* [nh*2d][H] ([q|gate] per head) */
    const uint16_t *wk, *wv;        /* [nkv*d][H] */
    const uint16_t *wo;             /* [H][nh*d] */
} ApusHipAttnProj;

/* GDN layer decode / verify with its projections (c/layer.h:236-286 per
 * token): ln1 [Ttot][H] -> ao [Ttot][H]; the state arguments as
 * apus_hip_gdn_decode / _decode_slots. The four input projections (w_qkv,
 * w_z, w_b, w_a, c/layer.h:250-253) run as one MFMA GEMM launch whose
 * epilogue writes qkv, z, b, a in the mixer's layouts; then the fused
 * decode mixer; then w_out (c/layer.h:274). The GEMMs are the tolerance
 * class of apus_hip_bf16_gemm_mfma_dev; with the same projections the
 * mixer is bitwise apus_hip_gdn_decode. Needs hidden, value_dim and hv
 * multiples of 32. Library scratch holds the intermediates. */
int apus_hip_gdn_layer_decode(const ApusHipGdnLayer *L, const ApusHipGdnProj *P,
                              size_t B, const int32_t *cu, const uint16_t *ln1,
                              uint16_t *conv_state, float *S, uint16_t *ao);
int apus_hip_gdn_layer_decode_slots(const ApusHipGdnLayer *L, const ApusHipGdnProj *P,
                                    size_t B, const int32_t *slot_in,
                                    const int32_t *slot_out, const int32_t *cu,
                                    const uint16_t *ln1, uint16_t *conv, float *S,
                                    uint16_t *ao);
/* Full-attention layer decode / verify with its projections (c/layer.h:
 * 288-331 per token): wq | wk | wv as one MFMA GEMM launch writing qg, k, v
 * (c/layer.h:300-302), the split-K decode mixer on the flat or paged cache
 * (arguments as apus_hip_attn_decode / _decode_paged), then wo
 * (c/layer.h:322). */
int apus_hip_attn_layer_decode(const ApusHipAttnLayer *L, const ApusHipAttnProj *P,
                               size_t B, const int32_t *cu, const int32_t *pos0,
                               const uint16_t *ln1, uint16_t *kcache,
                               uint16_t *vcache, size_t max_seq, uint16_t *ao);
int apus_hip_attn_layer_decode_paged(const ApusHipAttnLayer *L, const ApusHipAttnProj *P,
                                     size_t B, const int32_t *rows, const int32_t *cu,
                                     const int32_t *pos0, const uint16_t *ln1,
                                     const ApusHipKvCache *kv, uint16_t *ao);

#ifdef __cplusplus
}
#endif
#endif /* APUS_HIP_H */
