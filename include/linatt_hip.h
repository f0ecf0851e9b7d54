/* linatt_hip: C ABI of the MI355X (gfx950) KATA-SPD / delta-rule kernels.
 *
 * All tensors are device pointers to contiguous, time-major arrays
 * (batch, time, head, feature).  The caller owns every buffer, including
 * workspaces sized by the *_workspace_bytes functions; the library never
 * allocates or frees device memory.  Every call is asynchronous on the
 * given HIP stream (`stream` is a hipStream_t; NULL means the null stream)
 * and never synchronises the device.  Functions return LINATT_OK (0) or a
 * negative status; linatt_last_error() then holds a message for the calling
 * thread.  No C++ exception crosses this boundary.
 *
 * dtype: LINATT_FLOAT32, LINATT_BFLOAT16 or LINATT_FLOAT16, shared by every
 * floating-point tensor of a call except den / delta / c (always float32).
 */
#ifndef LINATT_HIP_H
#define LINATT_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LINATT_ABI_VERSION 3

enum linatt_dtype { LINATT_FLOAT32 = 0, LINATT_BFLOAT16 = 1, LINATT_FLOAT16 = 2 };
enum linatt_kata_variant { LINATT_KATA_CONCAT = 0, LINATT_KATA_SUM = 1 };
/* OR-ed into the variant of the linatt_kata_gen_* calls: the packed state
 * layout (one row per unordered pair a <= b). */
enum { LINATT_KATA_PACKED_STATE = 4 };
enum linatt_status {
  LINATT_OK = 0,
  LINATT_EINVAL = -1,       /* null pointer, bad shape or misalignment */
  LINATT_EUNSUPPORTED = -2, /* valid, but no kernel is compiled for it */
  LINATT_ELAUNCH = -3       /* the HIP runtime rejected a launch */
};

/* ABI version of the loaded library (LINATT_ABI_VERSION at build time). */
int linatt_abi_version(void);

/* Message describing the last failed call on this thread ("" if none). */
const char* linatt_last_error(void);

/* 1 if a kernel is compiled for this combination, else 0.  No device work. */
int linatt_kata_supported(int dtype, int dk, int dv, int num_groups, int variant, int decay);

/* KATA-SPD causal attention forward.
 * Replaces the launch in parallel_kata_attn_fwd_impl
 * (kata/parallel_kata_attn.py:211-288; kernel kata/kernels/parallel_kata.py:8-197)
 * and parallel_kata_attn_sum_fwd_impl (kata/parallel_kata_attn.py:539-576;
 * kernel kata/kernels/parallel_kata.py:200-345).
 *   q (B,T,HQ,dk), k (B,T,H,dk), v (B,T,H,dv)  [dtype]; HQ % H == 0 (GQA)
 *   c (B,T,HQ) float32 cumulative log-decay, or NULL (concat variant only)
 *   o (B,T,HQ,dv) [dtype], den (B,T,HQ) float32 = sum_{s<=t} A[t,s]
 *   scale multiplies each group dot before squaring (> 0).
 */
int linatt_kata_fwd(const void* q, const void* k, const void* v, const float* c, void* o,
                    float* den, int B, int T, int HQ, int H, int dk, int dv, int num_groups,
                    float scale, int variant, int dtype, void* stream);

/* Bytes of workspace linatt_kata_bwd needs: two (B, T, HQ) float32 arrays
 * (-<o, dO> and scale^2 / den per row) and, for LINATT_BFLOAT16, dO scaled by
 * scale^2 / den (B, T, HQ, dv_dim), which the dk/dv pass reads instead of dO.
 * ABI 3 added dv_dim and dtype. */
size_t linatt_kata_bwd_workspace_bytes(int B, int T, int HQ, int dv_dim, int dtype);

/* KATA-SPD causal attention backward: dq, dk, dv from q, k, v, o, den, dO.
 * Replaces parallel_kata_attn_bwd_triton (kata/parallel_kata_attn.py:364-529;
 * kernels kata/kernels/parallel_kata.py:348-1342) and
 * parallel_kata_attn_sum_bwd_triton_M{2,4} (kata/parallel_kata_attn.py:755-901;
 * kernels kata/kernels/parallel_kata_sum.py:7-825).  Unlike the reference it
 * also covers GQA (HQ = G*H) and every compiled M without a host fallback.
 *   dq (B,T,HQ,dk), dk (B,T,H,dk), dv (B,T,H,dv) [dtype], fully overwritten.
 *   workspace: linatt_kata_bwd_workspace_bytes(B,T,HQ,dv,dtype) bytes, 256-byte
 *   aligned.
 */
int linatt_kata_bwd(const void* q, const void* k, const void* v, const void* o,
                    const float* den, const void* dout, void* dq, void* dk, void* dv,
                    void* workspace, int B, int T, int HQ, int H, int dk_dim, int dv_dim,
                    int num_groups, float scale, int variant, int dtype, void* stream);

/* Backward of the decayed concat score A[t,s] * exp(min(c_t - c_s, 0)):
 * dq, dk, dv as linatt_kata_bwd plus dc (B,T,HQ) float32, the gradient of the
 * cumulative log-decay c.  Replaces the O(T^2)-memory autograd recompute of
 * _KataDecayFunction.backward (kata/parallel_kata_attn.py:313-347, through
 * _kata_decay_ref :291-310).  o, den come from linatt_kata_fwd with the same c.
 * Same workspace as linatt_kata_bwd. */
int linatt_kata_bwd_decay(const void* q, const void* k, const void* v, const float* c,
                          const void* o, const float* den, const void* dout, void* dq, void* dk,
                          void* dv, float* dc, void* workspace, int B, int T, int HQ, int H,
                          int dk_dim, int dv_dim, int num_groups, float scale, int dtype,
                          void* stream);

/* The two halves of linatt_kata_bwd, with its argument list, mirroring the
 * reference's separate dq and dk/dv launches (kata/parallel_kata_attn.py:488-528):
 * linatt_kata_bwd_dq writes dq and the per-row terms into workspace
 * (dk, dv may be NULL); linatt_kata_bwd_dkdv then reads workspace and writes
 * dk, dv (o, dq may be NULL).  Enqueue dq before dkdv on the same stream. */
int linatt_kata_bwd_dq(const void* q, const void* k, const void* v, const void* o,
                       const float* den, const void* dout, void* dq, void* dk, void* dv,
                       void* workspace, int B, int T, int HQ, int H, int dk_dim, int dv_dim,
                       int num_groups, float scale, int variant, int dtype, void* stream);
int linatt_kata_bwd_dkdv(const void* q, const void* k, const void* v, const void* o,
                         const float* den, const void* dout, void* dq, void* dk, void* dv,
                         void* workspace, int B, int T, int HQ, int H, int dk_dim, int dv_dim,
                         int num_groups, float scale, int variant, int dtype, void* stream);

/* KATA forward with the mixer's output RMSNorm fused into its epilogue.
 * Replaces the pair parallel_kata_attn(...) -> self.norm(o) of
 * KataAttention.forward (kata/layer.py:456-487, 539; the norm is
 * fla.modules.RMSNorm(head_v_dim, eps=norm_eps, dtype=float32), built at
 * :199-205).  Writes o and den exactly as linatt_kata_fwd, and also
 *   rstd (B,T,HQ) float32 = (mean_d o_r[d]^2 + eps)^-1/2,
 *   y (B,T,HQ,dv) [dtype]  = o_r * rstd * norm_weight   (norm_weight (dv)
 *   float32, or NULL for weight 1),
 * where o_r is o as stored (rounded to dtype), as the unfused norm reads it.
 * dk = dv = 64 in bfloat16 or float16 (else LINATT_EUNSUPPORTED); concat,
 * sum and decayed (c non-NULL) scores. */
int linatt_kata_fwd_onorm(const void* q, const void* k, const void* v, const float* c, void* o,
                          float* den, const float* norm_weight, float eps, void* y, float* rstd,
                          int B, int T, int HQ, int H, int dk, int dv, int num_groups, float scale,
                          int variant, int dtype, void* stream);

/* KATA forward's unnormalised numerator in float32:
 *   num (B,T,HQ,dv) float32 = sum_{s<=t} A[t,s] v_s  (= o * den, unrounded),
 *   den (B,T,HQ) float32 as linatt_kata_fwd.
 * Replaces the SPD delta rule's readout, whose kernel keeps its float32
 * accumulator (_readout_kernel, kata/spd/flash_delta.py:975-985, with the
 * sum score).  dk = dv = 64 in bfloat16 or float16. */
int linatt_kata_fwd_num(const void* q, const void* k, const void* v, float* num, float* den,
                        int B, int T, int HQ, int H, int dk, int dv, int num_groups, float scale,
                        int variant, int dtype, void* stream);

/* Bytes of workspace linatt_kata_bwd_onorm needs: linatt_kata_bwd's, then
 * per-workgroup partials of the norm-weight gradient. */
size_t linatt_kata_bwd_onorm_workspace_bytes(int B, int T, int HQ, int dv_dim, int dtype);

/* Backward of linatt_kata_fwd_onorm from dy, the gradient of y: the norm's
 * backward dO = rstd (w dy) - (rstd^3 / dv) <o, w dy> o (rounded to dtype, as
 * the unfused norm's dx) is formed in the dq pass's registers, then the
 * attention backward runs as linatt_kata_bwd (linatt_kata_bwd_decay when c
 * and dc are non-NULL).  dnorm_weight (dv) float32 = sum over rows of
 * dy * o * rstd, in a fixed order (may be NULL; requires norm_weight).  o,
 * den, rstd from linatt_kata_fwd_onorm with the same inputs.  bfloat16 at
 * dk = dv = 64 only.  Replaces the norm's backward and
 * parallel_kata_attn_bwd_triton (kata/parallel_kata_attn.py:364-529). */
int linatt_kata_bwd_onorm(const void* q, const void* k, const void* v, const float* c,
                          const void* o, const float* den, const float* rstd,
                          const float* norm_weight, const void* dy, void* dq, void* dk, void* dv,
                          float* dc, float* dnorm_weight, void* workspace, int B, int T, int HQ,
                          int H, int dk_dim, int dv_dim, int num_groups, float scale, int variant,
                          int dtype, void* stream);

/* Size of the fixed device scratch behind linatt_kata_bwd_noalloc (32 MiB). */
#define LINATT_NOALLOC_SCRATCH_BYTES (32u << 20)

/* linatt_kata_bwd without a workspace argument and without any allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results as linatt_kata_bwd; the
 * workspace comes from a fixed per-device array of
 * LINATT_NOALLOC_SCRATCH_BYTES inside the library (held from the first call
 * on a device until the process ends).  A call whose
 * linatt_kata_bwd_workspace_bytes(B, T, HQ, dv_dim, dtype) exceeds it returns
 * LINATT_EINVAL before any device work (bf16 config B8 T2048 HQ12 dv64 needs
 * 25.5 MiB).  Calls that overlap on one device share the array and race:
 * serialise them.  Calls no hipMalloc/hipFree. */
int linatt_kata_bwd_noalloc(const void* q, const void* k, const void* v, const void* o,
                            const float* den, const void* dout, void* dq, void* dk, void* dv,
                            int B, int T, int HQ, int H, int dk_dim, int dv_dim, int num_groups,
                            float scale, int variant, int dtype, void* stream);

/* LINATT_NOALLOC_SCRATCH_BYTES as compiled into the library. */
size_t linatt_noalloc_scratch_bytes(void);

/* ---------------------------------------------------------------------------
 * Chunked (gated) delta rule (DeltaNet / GatedDeltaNet), chunks of 64 tokens.
 * Replaces fla.ops.delta_rule.chunk_delta_rule and
 * fla.ops.gated_delta_rule.chunk_gated_delta_rule of the third-party package
 * flash-linear-attention==0.5.0 (pinned at scripts/setup.sh:27 of the
 * reference; reached through configs/model/200m/delta_net_200m.yaml:3 and
 * gated_deltanet_200m.yaml:4).
 *   q, k (B,T,H,dk), v (B,T,H,dv) [dtype]; beta, g (B,T,H) float32 (g is the
 *   per-token log decay, NULL for the ungated rule); h0, ht (B,H,dk,dv)
 *   float32, each optional (NULL: zero initial state / not returned).
 *   o (B,T,H,dv) [dtype].  scale multiplies q (> 0).
 * The forward fills `ctx` (linatt_delta_ctx_bytes) with what the backward
 * reads; keep it unchanged between the two calls.
 * ------------------------------------------------------------------------- */

/* 1 if a kernel is compiled for (dtype, dk, dv), else 0.  No device work. */
int linatt_delta_supported(int dtype, int dk, int dv);

/* Bytes of the forward context and of the backward scratch (0 on bad shape). */
size_t linatt_delta_ctx_bytes(int B, int T, int H, int dk, int dv, int dtype);
size_t linatt_delta_bwd_workspace_bytes(int B, int T, int H, int dk, int dv, int dtype);

/* Forward: o and (optionally) the final state ht. */
int linatt_delta_fwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* g, const float* h0, void* o, float* ht, void* ctx, int B,
                     int T, int H, int dk, int dv, float scale, int dtype, void* stream);

/* Backward for the loss <o, dout> + <ht, dht> (dht may be NULL): dq, dk, dv
 * [dtype], dbeta (B,T,H) float32, dg (B,T,H) float32 (required when g is
 * given), dh0 (B,H,dk,dv) float32 (optional).  Same inputs as the forward
 * plus its ctx; workspace: linatt_delta_bwd_workspace_bytes. */
int linatt_delta_bwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* g, const float* h0, const void* dout, const float* dht,
                     const void* ctx, void* workspace, void* dq, void* dk, void* dv,
                     float* dbeta, float* dg, float* dh0, int B, int T, int H, int dk_dim,
                     int dv_dim, float scale, int dtype, void* stream);

/* The two calls above, one kernel at a time, for timing each kernel apart
 * (no counterpart in the reference, whose fla ops are single calls).
 * `stages` selects the kernels to launch, in this order: forward bit 0 the
 * chunk-local prep, bit 1 the state pass (which also writes o); backward
 * bit 0 the reverse state pass, bit 1 the chunk kernel.  Running every bit
 * once, in order, on one stream equals the full call. */
int linatt_delta_fwd_stages(const void* q, const void* k, const void* v, const float* beta,
                            const float* g, const float* h0, void* o, float* ht, void* ctx, int B,
                            int T, int H, int dk, int dv, float scale, int stages, int dtype,
                            void* stream);
int linatt_delta_bwd_stages(const void* q, const void* k, const void* v, const float* beta,
                            const float* g, const float* h0, const void* dout, const float* dht,
                            const void* ctx, void* workspace, void* dq, void* dk, void* dv,
                            float* dbeta, float* dg, float* dh0, int B, int T, int H, int dk_dim,
                            int dv_dim, float scale, int stages, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * KATA-SPD psi-state form: long-context prefill and recurrent decode.
 * psi(x) = vec(x_g x_g^T) per group (full E^2 rows, p = g E^2 + a E + b),
 * state S = sum_s psi(sqrt(scale) k_s) v_s^T (B,H,M*E^2,dv) float32 and
 * z = sum_s psi(sqrt(scale) k_s) (B,H,M*E^2) float32.
 * ------------------------------------------------------------------------- */

/* State form of every flash score, for decoding (no reference counterpart:
 * the reference's flash branch keeps no state, kata/layer.py:492).  Features
 *   concat (variant 0): psi(x)_p = scale x[gE+a] x[gE+b],  p = g E^2 + a E + b,
 *                       P = num_groups E^2  (kata/parallel_kata_attn.py:49-75)
 *   sum (variant 1):    psi(x)_p = scale sum_g x[gE+a] x[gE+b],  p = a E + b,
 *                       P = E^2  (the sum score, :539-576)
 * with E = dk / num_groups a power of two >= 16, dk <= 128, dv = 64; state
 * S (B,H,P,64) and z (B,H,P) float32.  c is the cumulative log-decay of the
 * decayed score (:291-310) within the call (each call's c starts from the
 * stored state at 0), non-increasing; NULL for no decay.
 *   S_t = e^(c_t - c_{t-1}) S_{t-1} + psi(k_t) v_t^T,  z likewise,
 *   o_t = psi(q_t)^T S_t / max(psi(q_t) . z_t, eps).
 * variant | LINATT_KATA_PACKED_STATE keeps the state packed: psi's rows
 * (a, b) and (b, a) are equal, so one row per pair a <= b of each group,
 *   p = g TE + a E - a (a - 1) / 2 + (b - a),  TE = E (E + 1) / 2,
 * P = num_groups TE (concat) or TE (sum); each row equals the full layout's
 * row (a, b), and the readouts count an off-diagonal row twice. */

/* Rows P of the state for (dk, num_groups, variant); 0 on bad arguments. */
int linatt_kata_gen_state_rows(int dk, int num_groups, int variant);

/* One decode step per (b, h): q, k (B,H,dk), v, o (B,H,64) [dtype]; c (B,H)
 * float32 the step's log-decay or NULL; S, z updated in place. */
int linatt_kata_gen_decode(const void* q, const void* k, const void* v, const float* c, float* S,
                           float* z, void* o, int B, int H, int dk, int dv, int num_groups,
                           int variant, float scale, float eps, int dtype, void* stream);

/* No reference counterpart; for serving at small batch.  The same decode
 * step with each (b, h)'s state rows split over several workgroups (about
 * 768 workgroups in all, at least 64 rows each; states of fewer than 512 rows
 * are not split), whose partial sums a second
 * launch adds in a fixed order: B*H (b, h) pairs then fill the chip instead
 * of walking their rows on B*H workgroups.  workspace (16-byte aligned) holds
 * linatt_kata_gen_decode_workspace_bytes bytes, 0 when no split pays (the
 * workspace may then be NULL).  Same results as linatt_kata_gen_decode up to
 * the order of the final fp32 sums. */
size_t linatt_kata_gen_decode_workspace_bytes(int B, int H, int dk, int num_groups, int variant);
int linatt_kata_gen_decode_split(const void* q, const void* k, const void* v, const float* c,
                                 float* S, float* z, void* o, void* workspace,
                                 size_t workspace_bytes, int B, int H, int dk, int dv,
                                 int num_groups, int variant, float scale, float eps, int dtype,
                                 void* stream);

/* A prefill continued from a state: o (B,T,H,64) [dtype] and den (B,T,H)
 * float32 hold the flash forward (linatt_kata_fwd) over the call's tokens on
 * entry; on return o = (o den + e^{c_t} psi(q_t)^T S) / max(den', eps) with
 * den' = den + e^{c_t} psi(q_t) . z, and den = max(den', eps).  q (B,T,H,dk);
 * c (B,T,H) or NULL; S, z are read only; q, S and o 16-byte aligned.
 * 16-bit inputs: psi(q_t)^T S runs on the matrix cores with psi(q_t) and S
 * rounded to bfloat16 and float32 sums; den stays float32. */
int linatt_kata_gen_readout(const void* q, const float* c, const float* S, const float* z,
                            void* o, float* den, int B, int T, int H, int dk, int dv,
                            int num_groups, int variant, float scale, float eps, int dtype,
                            void* stream);

/* The state after the call's tokens: S <- (init ? e^{c_T} S : 0) +
 * sum_s e^{c_T - c_s} psi(k_s) v_s^T, z likewise; k (B,T,H,dk), v (B,T,H,64),
 * c (B,T,H) or NULL; S, z updated in place; k, v and S 16-byte aligned.
 * 16-bit inputs: the products psi(k_s) v_s^T run on the matrix cores with
 * psi(k_s) (formed in float32) and v_s rounded to bfloat16, accumulated in
 * float32; z adds the float32 features; float32 inputs stay float32. */
int linatt_kata_gen_update(const void* k, const void* v, const float* c, float* S, float* z,
                           int init, int B, int T, int H, int dk, int dv, int num_groups,
                           int variant, float scale, int dtype, void* stream);

/* 1 if the state-form kernels are compiled for the combination, else 0. */
int linatt_kata_state_supported(int dtype, int dk, int dv, int num_groups);

/* Bytes of scratch linatt_kata_prefill needs. */
size_t linatt_kata_prefill_workspace_bytes(int B, int T, int H, int dk, int dv, int num_groups,
                                           int seg_len, int dtype);

/* Causal KATA forward in O(T) state form, plus the state after the last token.
 * Replaces spd_chunk_scan_cat (kata/spd/chunk_scan_cat.py:219-345): same output
 * o = num / max(den, eps) with den = sum_{s<=t} scale^2 sum_g (q_g.k_g)^2.
 * T is split into segments of seg_len tokens (a multiple of 128): psi states
 * across segments, the quadratic score inside a segment.
 *   head_major = 1: q, k (B,H,T,dk), v, o (B,H,T,dv), den (B,H,T)  (reference layout)
 *   head_major = 0: q, k (B,T,H,dk), v, o (B,T,H,dv), den (B,T,H)
 *   S_out, z_out may be NULL. */
int linatt_kata_prefill(const void* q, const void* k, const void* v, void* o, float* den,
                        float* S_out, float* z_out, void* workspace, int B, int T, int H, int dk,
                        int dv, int num_groups, float scale, float eps, int seg_len,
                        int head_major, int dtype, void* stream);

/* linatt_kata_prefill continued from a state: S_in (B,H,M*E^2,dv) and z_in
 * (B,H,M*E^2) float32 (both NULL: zero state) hold the state after the
 * tokens before q's first one; every output, and S_out / z_out, then covers
 * those tokens too.  S_out / z_out may alias S_in / z_in (in-place update).
 * The prefill a past_key_values cache needs to append a chunk of tokens to a
 * state (the reference keeps none for its flash path, kata/layer.py:492). */
int linatt_kata_prefill_state(const void* q, const void* k, const void* v, void* o, float* den,
                              const float* S_in, const float* z_in, float* S_out, float* z_out,
                              void* workspace, int B, int T, int H, int dk, int dv, int num_groups,
                              float scale, float eps, int seg_len, int head_major, int dtype,
                              void* stream);

/* The linear feature of the same tree-scan, spd_chunk_scan_cat(...,
 * feature="linear") (kata/spd/chunk_scan_cat.py:219-345): psi(x) =
 * sqrt(scale) x per group, so kappa(q, k) = scale (q . k) whatever the group
 * split, den_t = max(sum_{s<=t} kappa(q_t, k_s), eps) (it may be negative
 * before the clamp) and o_t = sum_{s<=t} kappa(q_t, k_s) v_s / den_t.
 * Head-major q, k (B,H,T,d), v, o (B,H,T,dv) [dtype], den (B,H,T) float32;
 * d = dv = 64, bf16 or fp16.  A chunked state pass (64-token chunks, state
 * k^T v in float32, one workgroup per (b, h)). */
int linatt_linear_scan_fwd(const void* q, const void* k, const void* v, void* o, float* den, int B,
                           int H, int T, int d, int dv, float scale, float eps, int dtype,
                           void* stream);

/* One recurrent decode token per (b, h): S += psi(sqrt(scale) k) v^T,
 * z += psi(sqrt(scale) k), o = psi(sqrt(scale) q)^T S / max(psi(sqrt(scale) q).z, eps).
 * q, k (B,H,dk), v, o (B,H,dv); S, z updated in place.  No reference
 * counterpart: the reference's flash path keeps no decode state
 * (kata/layer.py:492; eval_recall.py:133-144). */
int linatt_kata_decode_step(const void* q, const void* k, const void* v, float* S, float* z,
                            void* o, int B, int H, int dk, int dv, int num_groups, float scale,
                            float eps, int dtype, void* stream);

/* The same state in the packed layout.  psi(x)_g = vec(x_g x_g^T) is
 * symmetric in (a, b), so the packed state keeps one row per unordered pair
 * a <= b of each group: row g E (E + 1) / 2 + a E - a (a - 1) / 2 + (b - a)
 * holds what rows g E^2 + a E + b and g E^2 + b E + a of the full layout
 * both hold (E = dk / num_groups).  S (B,H,M E (E + 1) / 2,dv), z
 * (B,H,M E (E + 1) / 2) float32: 136 of 256 rows per group at M = 4, so a
 * decode step moves about half the bytes.  Outputs equal the full-layout
 * calls', and the states hold the same values (the pair's rows).  No
 * reference counterpart (the reference keeps no decode state); for
 * callers that keep a state between calls (decode caches, serving). */
int linatt_kata_prefill_state_packed(const void* q, const void* k, const void* v, void* o,
                                     float* den, const float* S_in, const float* z_in, float* S_out,
                                     float* z_out, void* workspace, int B, int T, int H, int dk,
                                     int dv, int num_groups, float scale, float eps, int seg_len,
                                     int head_major, int dtype, void* stream);
int linatt_kata_decode_step_packed(const void* q, const void* k, const void* v, float* S, float* z,
                                   void* o, int B, int H, int dk, int dv, int num_groups,
                                   float scale, float eps, int dtype, void* stream);

/* No reference counterpart; for serving at small batch.  linatt_kata_decode_step
 * (packed = 0) or _packed (packed = 1) with each (b, h)'s state rows split
 * over several workgroups (about 768 in all, at least 64 rows each), their
 * partial sums added in a fixed order by a second launch; workspace (16-byte
 * aligned) holds linatt_kata_decode_workspace_bytes bytes (0: no split; the
 * workspace may then be NULL).  Same results up to the order of the final
 * fp32 sums. */
size_t linatt_kata_decode_workspace_bytes(int B, int H, int dk, int num_groups, int packed);
int linatt_kata_decode_step_split(const void* q, const void* k, const void* v, float* S, float* z,
                                  void* o, void* workspace, size_t workspace_bytes, int B, int H,
                                  int dk, int dv, int num_groups, int packed, float scale, float eps,
                                  int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * SPD delta rule (DeltaKata).  Replaces the forward of flash_delta
 * (kata/spd/flash_delta.py:1060-1116: _flash_U_kernel :25-183,
 * _readout_kernel :898-972, _den_kernel :986-1046), called by the mixer's
 * delta branch (kata/layer.py:377-420).  With the sum-SPD kernel
 * kappa(a, b) = sum_{g,h} (scale a_g . b_h)^2 (the reference's sqrt(scale)
 * on q and on k):
 *   U = (I + diag(beta) strict_lower(kappa(k, k)))^-1 diag(beta) V,
 *   den_t = sum_{s<=t} kappa(q_t, k_s),  num = lower(kappa(q, k)) U,
 *   o = normalize ? num / (den + eps) : num.
 *   q, k (B,T,H,d), v (B,T,H,dv) [dtype]; beta (B,T,H) float32;
 *   U (B,T,H,dv) float32 (may be NULL), o (B,T,H,dv) float32, den (B,T,H) float32.
 * workspace: linatt_dkata_workspace_bytes. */
int linatt_dkata_supported(int dtype, int d, int dv, int num_groups);
size_t linatt_dkata_workspace_bytes(int B, int T, int H, int d, int dv, int dtype);
int linatt_dkata_fwd(const void* q, const void* k, const void* v, const float* beta, float* U,
                     float* o, float* den, void* workspace, int B, int T, int H, int d, int dv,
                     int num_groups, float scale, int normalize, float eps, int dtype,
                     void* stream);

/* The forward for training: as linatt_dkata_fwd (U may be NULL: the
 * backward reads the workspace's 16-bit copy of U, not U); the workspace
 * then also holds what linatt_dkata_bwd reads and must reach it unchanged. */
int linatt_dkata_fwd_train(const void* q, const void* k, const void* v, const float* beta,
                           float* U, float* o, float* den, void* workspace, int B, int T, int H,
                           int d, int dv, int num_groups, float scale, int normalize, float eps,
                           int dtype, void* stream);

/* Backward, replacing flash_delta_bwd (kata/spd/flash_delta.py:830-895) and
 * _FlashDelta.backward (:1084-1108): dq, dk (B,T,H,d), dv (B,T,H,dv) [dtype]
 * and dbeta (B,T,H) float32 for the loss <o, dout> (dout float32, the
 * forward's output dtype).  o (normalize only), den: the training
 * forward's outputs (U is not read and may be NULL; it stays in the list
 * the reference's backward saves); fwd_workspace: its workspace; workspace:
 * linatt_dkata_bwd_workspace_bytes.  bfloat16 only (fp16 cannot carry the
 * intermediate dU at small scales); other dtypes return LINATT_EUNSUPPORTED. */
size_t linatt_dkata_bwd_workspace_bytes(int B, int T, int H, int d, int dv, int dtype);
int linatt_dkata_bwd(const void* q, const void* k, const void* v, const float* beta,
                     const float* U, const float* o, const float* den, const float* dout,
                     void* dq, void* dk, void* dv, float* dbeta, void* fwd_workspace,
                     void* workspace, int B, int T, int H, int d, int dv_dim, int num_groups,
                     float scale, int normalize, float eps, int dtype, void* stream);

/* ---------------------------------------------------------------------------
 * Token-mixer prologue / epilogue (the non-GEMM ops around the attention op
 * in kata/layer.py KataAttention.forward).
 *
 * Causal depthwise short convolution with optional SiLU, replacing
 * fla.modules.ShortConvolution as the mixer uses it (kata/layer.py:178-197,
 * 299-318; third-party flash-linear-attention==0.5.0, absent here):
 *   z[b,t,c] = bias[c] + sum_{w<W} weight[c,w] x[b, t-(W-1)+w, c],
 *   y = activation ? silu(z) : z.
 * x, y (B,T,C) [dtype], C a multiple of 8, W in {2,3,4}; weight (C,W) and
 * bias (C) float32 (bias may be NULL).  cache_in (B,C,W) [dtype]: the W inputs
 * before position 0, newest last (NULL: zeros); cache_out (B,C,W): the W
 * inputs before position T, for the next call (may be NULL; it may alias
 * cache_in only when T <= 16, else LINATT_EINVAL).  The backward
 * gives dx and float32 dweight (C,W) / dbias (C, may be NULL); no gradient
 * flows to cache_in.  Workspace: linatt_short_conv_bwd_workspace_bytes. */
int linatt_short_conv_fwd(const void* x, const float* weight, const float* bias,
                          const void* cache_in, void* y, void* cache_out, int B, int T, int C,
                          int W, int activation, int dtype, void* stream);
size_t linatt_short_conv_bwd_workspace_bytes(int B, int T, int C, int W);
int linatt_short_conv_bwd(const void* x, const float* weight, const float* bias,
                          const void* cache_in, const void* dy, void* dx, float* dweight,
                          float* dbias, void* workspace, int B, int T, int C, int W,
                          int activation, int dtype, void* stream);

/* Rotary position embedding, replacing fla.modules.RotaryEmbedding as the
 * mixer uses it (kata/layer.py:130-148, 352-372): x, y (B,T,H,D) [dtype]
 * (y may equal x); pair p of the first rot_dim dims -- (2p, 2p+1) if
 * interleaved, else (p, p + rot_dim/2) -- is rotated by the angle
 * (t + offset) * base^(-2p/rot_dim) computed in fp32; inverse != 0 rotates
 * the other way (the backward).  Dims past rot_dim are copied. */
int linatt_rope(const void* x, void* y, int B, int T, int H, int D, int rot_dim, float base,
                int offset, int interleaved, int inverse, int dtype, void* stream);

/* Fused q/k prologue: the short convolution + activation, the per-head norm
 * and the rotary embedding in one pass.  It replaces the chain that
 * kata/layer.py:305-318, 345-372 runs on q and on k as three modules
 * (ShortConvolution -> RMSNorm(head_k_dim, fp32 weight) or l2norm ->
 * RotaryEmbedding), with the intermediates kept in fp32 instead of rounded to
 * the input dtype between the modules:
 *   u = act(bias + sum_w conv_weight[c,w] x[b, t-(W-1)+w, c])   (as
 *       linatt_short_conv_fwd, with cache_in / cache_out, which may alias
 *       only when T <= 16),
 *   norm 1: n = u (mean_d u^2 + eps)^-1/2 norm_weight (norm_weight NULL: 1);
 *   norm 2: n = u (sum_d u^2 + eps)^-1/2 (fla l2norm; norm_weight must be
 *           NULL); norm 0: n = u;
 *   y = n rotated as linatt_rope rotates each row of rope_width dims (the
 *       head dim D for full-head RoPE, the group width E for rope_group) over
 *       its first rot_dim dims, positions offset .. offset + T - 1;
 *       rot_dim 0: no rotation.
 * x, y (B,T,H*D) [dtype] (y is (B,T,H,D)); conv_weight (H*D,W), conv_bias
 * (H*D) or NULL, norm_weight (D): float32.  D in {32, 64, 128}, W in
 * {2,3,4}; rope_width a multiple of 4 dividing D; rot_dim even and at most
 * rope_width, a multiple of 8 when not interleaved.  The backward gives dx
 * and float32 dconv_weight (H*D,W), dconv_bias (H*D, may be NULL),
 * dnorm_weight (D, may be NULL); no gradient flows to cache_in.
 * Workspace: linatt_qk_prologue_bwd_workspace_bytes. */
int linatt_qk_prologue_fwd(const void* x, const float* conv_weight, const float* conv_bias,
                           const void* cache_in, const float* norm_weight, void* y,
                           void* cache_out, int B, int T, int H, int D, int W, int activation,
                           int norm, float eps, int rope_width, int rot_dim, float base,
                           int offset, int interleaved, int dtype, void* stream);
size_t linatt_qk_prologue_bwd_workspace_bytes(int B, int T, int H, int D, int W);
int linatt_qk_prologue_bwd(const void* x, const float* conv_weight, const float* conv_bias,
                           const void* cache_in, const float* norm_weight, const void* dy,
                           void* dx, float* dconv_weight, float* dconv_bias, float* dnorm_weight,
                           void* workspace, int B, int T, int H, int D, int W, int activation,
                           int norm, float eps, int rope_width, int rot_dim, float base,
                           int offset, int interleaved, int dtype, void* stream);

/* RMSNorm over the last dim of a contiguous (n, d) array, fp32 arithmetic,
 * replacing fla.modules.RMSNorm as the mixer uses it (output norm
 * kata/layer.py:199-205, 539; q/k norm :126-128, 347):
 *   y = x r weight, r = (mean(x^2) + eps)^-1/2 (rstd (n) float32 saved);
 * weight (d) float32 or NULL (no affine).  d = 8 times a power of two, at
 * most 512.  Backward: dx and, with weight, dweight (d) float32.
 * Workspace: linatt_rmsnorm_bwd_workspace_bytes. */
int linatt_rmsnorm_fwd(const void* x, const float* weight, void* y, float* rstd, int n, int d,
                       float eps, int dtype, void* stream);
size_t linatt_rmsnorm_bwd_workspace_bytes(int n, int d);
int linatt_rmsnorm_bwd(const void* x, const float* weight, const float* rstd, const void* dy,
                       void* dx, float* dweight, void* workspace, int n, int d, int dtype,
                       void* stream);

/* Row L2 normalisation over the last dim of a contiguous (n, d) array:
 * y = x / sqrt(sum x^2 + eps), rstd (n) float32 = 1 / sqrt(sum x^2 + eps);
 * backward dx = rstd (dy - y <y, dy>).  The normalisation fla applies to q
 * and k under use_qk_l2norm_in_kernel=True (DeltaNet configs set
 * qk_norm: l2, configs/model/200m/delta_net_200m.yaml:13). */
int linatt_l2norm_fwd(const void* x, void* y, float* rstd, int n, int d, float eps, int dtype,
                      void* stream);
int linatt_l2norm_bwd(const void* y, const float* rstd, const void* dy, void* dx, int n, int d,
                      int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LINATT_HIP_H */
