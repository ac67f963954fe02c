/* irontimber-mi355x: C ABI of the attention / Gated-DeltaNet hot path, hand-written HIP for gfx950.
 *
 * Conventions (all entry points):
 *   - Every pointer argument is a device pointer unless its comment says otherwise. The caller owns
 *     every buffer (inputs, outputs, KV cache, recurrent state, scratch); the library allocates and
 *     frees nothing. (The reference's Vulkan backend follows the same rule with one caller-owned
 *     arena: src/vk/mod.rs:2-6, 544-566.)
 *   - `stream` is a hipStream_t (NULL = the legacy default stream). Calls only enqueue work; they
 *     do not synchronise.
 *   - Return 0 on success. A nonzero return means nothing was enqueued (geometry, alignment or
 *     scratch validation failed on the host) or a launch failed; it_last_error() then returns a
 *     thread-local message. This mirrors the reference's Result<(), String> validation before any
 *     device work (src/vk/mod.rs:179-220).
 *   - Strides are counted in elements of the pointed-to type.
 *   - Calls on one stream from one thread, like the reference's !Sync Ctx (src/vk/mod.rs:235-240).
 */
#ifndef IT_ATTN_H
#define IT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Thread-local text of the last error (empty string if none). */
const char* it_last_error(void);

/* ABI version: bumped whenever a signature or a buffer layout below changes. */
int it_abi_version(void);

/* ------------------------------------------------------------------------------------------------
 * Softmax attention over an f16 KV cache (decode, MTP verify, chunked and whole-prompt prefill).
 * ---------------------------------------------------------------------------------------------- */

/* Append nt new K and V rows (f32, already RMS-normed and roped) to the f16 cache at rows
 * pos0..pos0+nt-1. Source row t is k[t*src_tok_stride + i], i < kvd. Cache row p is kc[p*kvd + i].
 * round_mode 0 = round to nearest even (the half crate's f16::from_f32 used by cpu.rs:22),
 * 1 = round toward zero (packHalf2x16 on the reference's HAWAII GPU, src/vk/r012_parity.rs:14-18).
 * Replaces the pair of kv_pack dispatches, src/vk/mod.rs:832-838 (kernel kernels/src/lib.rs:743-750). */
int it_kv_append_f16(const float* k, const float* v, int src_tok_stride, uint16_t* kc, uint16_t* vc,
                     int pos0, int nt, int kvd, int round_mode, void* stream);

/* The whole pre-attention pass in one launch: per-head RMSNorm of q and k, neox-style (I)MRoPE on
 * the first n_rot dims of each q and k head at positions pos0+t, and the f16 append of K and V.
 *   q      : f32 [t*q_tok_stride + h*2*hd + d]; d < hd (the query) is rewritten in place with
 *            rope(rmsnorm(q) * q_norm); d in [hd, 2hd) (the gate) is left as it is.
 *   k, v   : f32 [t*kv_tok_stride + kh*hd + d], the k and v projections (read only).
 *   kc, vc : f16 cache rows pos0+t receive f16(rope(rmsnorm(k) * k_norm)) and f16(v).
 *   q_norm, k_norm: f32 [hd] weights, or NULL for unit weight. eps: the RMSNorm epsilon.
 *   n_rot  : rotated dims per head (even, <= hd, a multiple of hd/32); theta_scale the f32
 *            base^(-2/n_rot) the reference pushes (src/vk/mod.rs:824); sec0..sec3 the rope
 *            sections (a frequency outside the text sections keeps angle 0, cpu.rs:152-155).
 *   round_mode as for it_kv_append_f16. hd is 128 or 256.
 * The angles p*theta_scale^i are formed in f64, so they are exact to f32 rounding at any position.
 * Replaces the six dispatches of src/vk/mod.rs:822-838 (two rmsnorm mode 0, two rope, two kv_pack;
 * kernels/src/lib.rs:207-229, 233-250, 743-750) and cpu.rs:249-258. */
int it_attn_prep_f16(float* q, int q_tok_stride, const float* k, const float* v, int kv_tok_stride,
                     const float* q_norm, const float* k_norm, float eps, uint16_t* kc, uint16_t* vc, int kvd,
                     int pos0, int hd, int nh, int nkv, int nt, int n_rot, float theta_scale, int sec0, int sec1,
                     int sec2, int sec3, int round_mode, void* stream);

/* it_attn_prep_f16 that also writes the query in the form the flash prefill kernel computes with:
 * q16[t*q16_tok_stride + h*hd + d] = f16_rne(q'[d] * (scale * log2(e))), q' the rewritten query
 * and scale the attention scale the following it_attn_f16_q16 call will pass (the product taken
 * in f32, as that kernel takes it). q16: 16-byte aligned f16 (uint16_t bits), q16_tok_stride a
 * multiple of 8, >= nh*hd. No counterpart in the reference (its prefill kernels read f32 q): an
 * opt-in for prefill callers, whose flash kernel then reads half the q bytes and no f32 rows. */
int it_attn_prep_f16_q16(float* q, int q_tok_stride, const float* k, const float* v, int kv_tok_stride,
                         const float* q_norm, const float* k_norm, float eps, uint16_t* kc, uint16_t* vc, int kvd,
                         int pos0, int hd, int nh, int nkv, int nt, int n_rot, float theta_scale, int sec0, int sec1,
                         int sec2, int sec3, int round_mode, uint16_t* q16, int q16_tok_stride, float scale,
                         void* stream);

/* Bytes of scratch it_attn_f16 needs for this call geometry (0 if the chosen kernel needs none). */
size_t it_attn_scratch_bytes(int pos0, int nt, int hd, int nh, int nkv);

/* Causal GQA attention with sigmoid output gate, f32 accumulation.
 *   q    : f32. Token t, q-head h: q[t*q_tok_stride + h*2*hd + d] for d < hd is the (normed, roped)
 *          query and d in [hd, 2hd) the output gate (the reference's q row, cpu.rs:249-254).
 *   kc,vc: f16 cache [pos][kvd], kvd = nkv*hd; KV head kh at column kh*hd. Rows 0..pos0+nt-1 must
 *          be written (append first with it_kv_append_f16).
 *   Token t attends keys 0..pos0+t (n = pos0+t+1, cpu.rs:260; kernels/src/lib.rs:764); q-head h
 *   reads KV head h/(nh/nkv) (cpu.rs:265).
 *   out  : f32 out[t*out_tok_stride + h*hd + d] = softmax(scale*q.K) V * sigmoid(gate).
 *   scratch: device buffer for the partial records (split-K: 260 f32 words per token, head and split;
 *          flash key splits: 132 words, O as int16). it_attn_scratch_bytes(...) bytes give the
 *          library's preferred split; with fewer bytes the keys per split double until the records
 *          fit (the reference's rule for its fixed arena, src/vk/mod.rs:714-716), and the prefill
 *          kernel falls back to one pass with no scratch. The reference's own room,
 *          it_attention_dispatch_room(ctx_len, nh, nt) * 4 bytes, is always enough. NULL = 0 bytes.
 * Requires hd == 256, nh % nkv == 0, q_tok_stride and out_tok_stride multiples of 4, 16-byte
 * aligned q/out/kc/vc (the reference asserts the same f16 layout, src/vk/mod.rs:713).
 * Replaces VkEngine::attention_kv(qo,qts,kco,vco,kvd,pos0,hd,nh,nkv,oo,nt,f16=true),
 * src/vk/mod.rs:710-729, i.e. the split-K partial dispatch plus attn_comb. One entry point covers
 * decode (nt=1), MTP verify (nt<=4), chunked prefill (nt=64, pos0>0) and whole-prompt prefill. */
int it_attn_f16(const float* q, int q_tok_stride, const uint16_t* kc, const uint16_t* vc, int kvd,
                int pos0, int hd, int nh, int nkv, int nt, float scale, float* out, int out_tok_stride,
                void* scratch, size_t scratch_bytes, void* stream);

/* it_attn_f16 with the kernel choice exposed (the reference's BONSAI_PREFILL_ATTN / chunk policy,
 * src/vk/mod.rs:714-717 and 192-204):
 *   kernel 0 = automatic (what it_attn_f16 does), 1 = split-K partials + combine,
 *          2 = flash prefill (any nt; the automatic choice from nt = 16): one pass with no scratch,
 *          or, when one pass would leave most of the GPU idle (a short chunk after a long context),
 *          key splits whose
 *          partial records (132 words: {m, l, k, 0} and O as int16 in units of k) are merged like
 *          kernel 1's,
 *          3 = kernel 2 with lossless key-split records: the split-K kernel's 260-word f32 form
 *          {m, l, 0, 0, o[256]} instead of int16 O (twice the scratch; the same result as one
 *          pass up to f32 reassociation of the merge).
 *   chunk  = keys per split, 0 = automatic: a multiple of 32 for kernel 1 (the automatic split is
 *          32 keys for 1-2 tokens below 2048 keys, else 64), of 64 for kernels 2 and 3, where a
 *          chunk of at least pos0 + nt means one pass.
 * it_attn_scratch_bytes_ex gives the scratch for the same choice. With chunk = 0 the split is fitted
 * to scratch_bytes as in it_attn_f16; an explicit chunk needs its full record set. */
size_t it_attn_scratch_bytes_ex(int pos0, int nt, int hd, int nh, int nkv, int kernel, int chunk);
int it_attn_f16_ex(const float* q, int q_tok_stride, const uint16_t* kc, const uint16_t* vc, int kvd,
                   int pos0, int hd, int nh, int nkv, int nt, float scale, float* out, int out_tok_stride,
                   void* scratch, size_t scratch_bytes, int kernel, int chunk, void* stream);

/* it_attn_f16 with the flash prefill kernel's query operand given pre-converted: q16 as written by
 * it_attn_prep_f16_q16 with the same scale (f16(q * scale * log2(e)), token stride q16_tok_stride).
 * The result is identical, bit for bit, to it_attn_f16 on the f32 q that q16 was made from; q
 * still provides the gates, and calls that take the split-K kernels (nt < 16) read q as
 * it_attn_f16 does. Same scratch rule and requirements as it_attn_f16. No counterpart in the
 * reference; see it_attn_prep_f16_q16. */
int it_attn_f16_q16(const float* q, int q_tok_stride, const uint16_t* q16, int q16_tok_stride, const uint16_t* kc,
                    const uint16_t* vc, int kvd, int pos0, int hd, int nh, int nkv, int nt, float scale, float* out,
                    int out_tok_stride, void* scratch, size_t scratch_bytes, void* stream);

/* it_attn_f16 that allocates nothing and takes no scratch argument. No counterpart in the reference:
 * it is for callers that cannot allocate device memory or hand over a workspace (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc). The partial records (split-K,
 * or the flash kernel's int16 key-split records) go to a file-scope device array of IT_NOALLOC_SCRATCH_BYTES (16 MiB) that each GPU the
 * library runs on holds until the process ends; the split is fitted to that size as for a caller
 * buffer of the same size (it_attn_plan(..., IT_NOALLOC_SCRATCH_BYTES, ...) gives the choice), and
 * a geometry whose records cannot fit (split-K with nt*nh*1040 bytes above the maximum) is rejected
 * with an error before any device work. Nothing in the array needs to start at zero: every record a
 * merge reads is written earlier in the same call. All calls on one GPU share that GPU's array, so
 * calls that overlap on one GPU (different streams, or graphs replayed concurrently) race; calls in
 * order on one stream do not. Other arguments and results as it_attn_f16. */
#define IT_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int it_attn_f16_noalloc(const float* q, int q_tok_stride, const uint16_t* kc, const uint16_t* vc, int kvd,
                        int pos0, int hd, int nh, int nkv, int nt, float scale, float* out, int out_tok_stride,
                        void* stream);

/* Decode attention in one launch. Replaces the same reference call as it_attn_f16 for decode
 * (VkEngine::attention_kv, src/vk/mod.rs:710-729: the attn_s_h partial dispatch and attn_comb,
 * kernels/src/lib.rs:722-798), with the split records and their merge in one kernel: each split
 * writes its record to a caller-owned mailbox, per 16 output dims, and the waves that merge a
 * (token, head, 16 dims) unit wait for exactly the pieces they read. Results are bit-identical to
 * it_attn_f16's. Slower than it_attn_f16 on MI355X (9.7 against 9.4 us per layer at ctx 8192),
 * and it relies on its whole grid being resident at once, so it_attn_f16 is the default; this
 * form is for a GPU the caller has to itself where one launch per layer matters. Taken when the geometry qualifies: a split-K call (nt < 16) with at most 8 query
 * rows per KV head (nt * nh / nkv <= 8: decode), at most 256 splits of 64 keys (pos0 + nt <= 16384)
 * and enough of them to give every (token, head, 16-dim block) merge a wave of its own (nt * nh *
 * 16 <= 4 * splits * nkv * row groups: with fewer, as at ctx 512, two launches are faster),
 * a mailbox of at least it_attn_mailbox_bytes(pos0 + nt, nt, nh) bytes, and a grid the device
 * holds at once (so every piece a merge waits for is being produced). Any other call runs
 * it_attn_f16 with `scratch` / `scratch_bytes`; it_attn_mailbox_would_launch reports which.
 *
 * The mailbox: 16-byte aligned device memory, initialised once with it_attn_mailbox_init and left
 * initialised by every call (each merge clears what it read). One mailbox serves any sequence of
 * calls in order on one stream (every layer and step of an engine); calls that overlap on the
 * device (other streams, concurrent graph replays) need one each. A merge that has waited 10 ms
 * (possible only if other work holds the device's compute units) gives up, writes NaN outputs and
 * poisons the mailbox: every later call then gives NaN at once until it_attn_mailbox_init runs
 * again. A mailbox that was never initialised (or was overwritten) is treated as poisoned too;
 * it_attn_mailbox_poisoned reports either. A merge that finds its mailbox poisoned also sets a
 * host-visible word that it_attn_mailbox_init allocates for the mailbox (pinned, one per mailbox,
 * kept until the process ends), so once such a call has completed, the next it_attn_f16_mailbox
 * call with that mailbox returns -1 ("poisoned", before any device work) instead of NaN again. */
size_t it_attn_mailbox_bytes(int ctx, int nt, int nh);
int it_attn_mailbox_init(void* mailbox, size_t bytes, void* stream);
int it_attn_mailbox_poisoned(const void* mailbox, int* poisoned, void* stream);   /* synchronises stream */
int it_attn_mailbox_would_launch(int pos0, int nt, int hd, int nh, int nkv, size_t mailbox_bytes);
int it_attn_f16_mailbox(const float* q, int q_tok_stride, const uint16_t* kc, const uint16_t* vc, int kvd,
                        int pos0, int hd, int nh, int nkv, int nt, float scale, float* out, int out_tok_stride,
                        void* mailbox, size_t mailbox_bytes, void* scratch, size_t scratch_bytes, void* stream);

/* The choice it_attn_f16 makes for this geometry and scratch budget: *kernel 1 (split-K) or 2
 * (flash), *chunk keys per split (0 = flash in one pass, no scratch), *bytes of scratch used.
 * Returns nonzero if no split fits (only possible for nt < 16 with fewer than nt*nh*1040 bytes).
 * Scratch per split: the split-K kernel's records are 260 f32 words per (token, head); the flash
 * kernel's key-split records are 132 words per (token, head): {m, l, k, 0} and O as int16 in
 * units of k = max|O| / 32767 (an error of at most max|O| / 65534 per value before the merge).
 * Host-only; the chunk loop is the reference's, src/vk/mod.rs:714-716. */
int it_attn_plan(int pos0, int nt, int hd, int nh, int nkv, size_t scratch_bytes, int* kernel, int* chunk,
                 size_t* bytes);

/* The two phases of the split-K path as separate calls (the reference dispatches them separately
 * too: attn_s_h then attn_comb, src/vk/mod.rs:725-727). Partial record of (token t, q-head h,
 * split s) is 260 floats {m, l, 0, 0, o[256]} at part + ((t*nh + h)*smax + s)*260 with
 * smax = ceil((pos0+nt)/chunk): m = max score, l = sum exp(score - m), o = sum exp(score - m) v
 * over the split's keys visible to token t (kernels/src/lib.rs:753-798). Records of splits a token
 * cannot see are never read (they are left untouched or written as {-inf, 0, 0, 0, 0...}). A sequence-sharded caller can exchange these records and run
 * it_attn_combine locally.
 *   it_attn_partials: part must hold it_attn_scratch_bytes_ex(pos0,nt,hd,nh,nkv,1,chunk) bytes.
 *   it_attn_combine : out = merge of the records of splits 0..ceil((pos0+t+1)/chunk)-1, times
 *                     sigmoid(gate) (kernels/src/lib.rs:722-740). */
int it_attn_partials(const float* q, int q_tok_stride, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                     int hd, int nh, int nkv, int nt, float scale, float* part, size_t part_bytes, int chunk,
                     void* stream);
int it_attn_combine(const float* q, int q_tok_stride, const float* part, int pos0, int hd, int nh, int nt, int chunk,
                    float* out, int out_tok_stride, void* stream);

/* The same two phases with a choice of record layout. layout 0: the 260-float records above (these
 * calls are then it_attn_partials / it_attn_combine). layout 1: the records it_attn_f16 itself
 * uses when its merge takes one wave per (token, head, 16 output dims), i.e. for 9-256 splits and
 * at most 256 (token, head) rows (decode and verify at long contexts; other geometries are
 * refused): the same f32 values, O as 64-byte pieces of 16 floats at
 * part + (((t*nh + h)*16 + d/16)*smax + s)*16 (+ d % 16), then {m, l} at
 * part + nt*nh*smax*256 + ((t*nh + h)*smax + s)*2, 1,032 bytes per (token, head, split) inside
 * the same part_bytes. The merge's lanes, one split each, then read adjacent pieces, which makes
 * the merge faster (ctx 8192: 8.45 against 9.0 us per layer); the output is bit-identical to
 * layout 0. Extends the reference's attn_s_h / attn_comb pair (kernels/src/lib.rs:722-798), which
 * has one layout only. */
int it_attn_partials_ex(const float* q, int q_tok_stride, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                        int hd, int nh, int nkv, int nt, float scale, float* part, size_t part_bytes, int chunk,
                        int layout, void* stream);
int it_attn_combine_ex(const float* q, int q_tok_stride, const float* part, int pos0, int hd, int nh, int nt, int chunk,
                       int layout, float* out, int out_tok_stride, void* stream);

/* ------------------------------------------------------------------------------------------------
 * The MTP head's attention over its own f32 KV cache (src/mtp.rs:96-130; src/vk/mod.rs:917-942).
 * Slot p of that cache holds position p + 1 (mtp.rs:120, vk/mod.rs:932).
 * ---------------------------------------------------------------------------------------------- */

/* it_attn_prep_f16 for an f32 cache: token t is roped at position pos0 + t and its normed, roped K
 * row and its V row are stored as f32 at cache row row0 + t (for the MTP head row0 = pos0 - 1).
 * Replaces the MTP pass's rmsnorm mode 0 (q_norm, k_norm) and rope dispatches, src/vk/mod.rs:933-938
 * (its k/v matvecs write the cache rows directly; here they write k, v and this call stores them). */
int it_attn_prep_f32kv(float* q, int q_tok_stride, const float* k, const float* v, int kv_tok_stride,
                       const float* q_norm, const float* k_norm, float eps, float* kc, float* vc, int kvd,
                       int pos0, int row0, int hd, int nh, int nkv, int nt, int n_rot, float theta_scale, int sec0,
                       int sec1, int sec2, int sec3, void* stream);

/* Bytes of scratch it_attn_f32kv prefers (split-K partial records, same 260-float layout: 64-key
 * splits for one block of up to 32 query rows per KV head, longer splits for multi-block calls);
 * any smaller scratch also works (it_attn_f32kv_plan). */
size_t it_attn_f32kv_scratch_bytes(int pos0, int nt, int hd, int nh, int nkv);

/* The split it_attn_f32kv uses for a scratch of scratch_bytes: *chunk keys per split and *bytes of
 * records, or *chunk = 0 and *bytes = 0 for the one-pass form that needs no scratch. The preferred
 * split is kept when it fits; otherwise the split doubles until the records fit, the reference's
 * rule for the MTP head's attention (src/vk/mod.rs:730-733, C doubling from 64 while
 * nt*nh*ceil((pos0+nt)/C)*260 words exceed the room); when even one record per (token, head) does
 * not fit it takes the one-pass form, as the reference falls back to its whole-context `attn`
 * kernel (src/vk/mod.rs:740, kernels/src/lib.rs:83-116). Returns 0, or -1 for a bad geometry. */
int it_attn_f32kv_plan(int pos0, int nt, int hd, int nh, int nkv, size_t scratch_bytes, int* chunk, size_t* bytes);

/* Causal GQA attention with sigmoid gate over an f32 KV cache: it_attn_f16's semantics and
 * buffers with kc, vc as f32 [row][kvd]. Query t sees cache rows 0..pos0+t (for the MTP head pass
 * pos0 is the first query's slot, position - 1). hd == 256, at most 16 q heads per KV head. The
 * split fits whatever scratch the caller passes (it_attn_f32kv_plan); a null scratch or one too
 * small for a record per (token, head) runs the one-pass form.
 * Replaces VkEngine::attention(..., f16 = false) for the MTP head, src/vk/mod.rs:707-709 and 942
 * (attn_s + attn_comb, kernels/src/lib.rs:682-740; CPU src/mtp.rs:122-130). */
int it_attn_f32kv(const float* q, int q_tok_stride, const float* kc, const float* vc, int kvd, int pos0, int hd,
                  int nh, int nkv, int nt, float scale, float* out, int out_tok_stride, void* scratch,
                  size_t scratch_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Gated DeltaNet: short causal conv, q/k L2 norm, gated-delta recurrence.
 * ---------------------------------------------------------------------------------------------- */

/* Depthwise causal conv (kernel K in 2..4) + SiLU over nt tokens, carrying the rolling (K-1)-token
 * state (oldest first) across calls.
 *   x     : f32 x[t*x_tok_stride + ch], ch < cd (the qkv projection output)
 *   w     : f32 w[ch*K + i]             (ssm_conv1d.weight)
 *   state : f32 state[i*cd + ch], i < K-1, updated in place to the last K-1 inputs
 *   out   : f32 out[t*out_tok_stride + ch]  (must not alias x or state)
 * Replaces the conv dispatch, src/vk/mod.rs:803 (kernel kernels/src/lib.rs:119-140; CPU
 * cpu.rs:201-212). */
int it_gdn_conv(const float* x, int x_tok_stride, const float* w, float* state, float* out,
                int out_tok_stride, int cd, int nt, int K, void* stream);

/* In-place L2 normalisation x / max(||x||, eps) of nheads consecutive rows of length d per token:
 * row r of token t is x[t*tok_stride + r*d ...]. d must be 128 or 256.
 * Replaces rmsnorm mode 2 on the 2*nk q/k heads, src/vk/mod.rs:804 (kernels/src/lib.rs:207-229;
 * cpu.rs:214). */
int it_l2norm_heads(float* x, int tok_stride, int nheads, int d, int nt, float eps, void* stream);

/* it_gdn_conv followed by it_l2norm_heads(out, ..., nnorm, 128, ...) in one pass: channels
 * [0, nnorm*128) (the q and k heads, nnorm = 2*nk) are L2-normalised per 128-channel head and token
 * after the conv + SiLU, the rest (v) are written as the conv gives them. Same buffers and state
 * rules as it_gdn_conv; cd must be a multiple of 128.
 * Replaces the conv and rmsnorm mode 2 dispatch pair, src/vk/mod.rs:803-804 (cpu.rs:201-214). */
int it_gdn_conv_l2norm(const float* x, int x_tok_stride, const float* w, float* state, float* out,
                       int out_tok_stride, int cd, int nt, int K, int nnorm, float eps, void* stream);

/* Gated-delta recurrence, token by token, for nt tokens (decode: nt=1).
 *   co    : f32 normalised conv output, token t at co[t*co_tok_stride]: q heads [0, nk*S),
 *           k heads [nk*S, 2*nk*S), v heads [2*nk*S, 2*nk*S + nv*S). V head h uses q/k head h % nk.
 *   beta_raw, alpha_raw: f32 [t*ba_tok_stride + h]; beta = sigmoid(beta_raw),
 *           g = softplus(alpha_raw + dt[h]) * a[h] (a < 0 is the decay rate), S <- exp(g) S.
 *   dt, a : f32 [nv]
 *   state : f32 [nv][S][S], element [h][i][j] = S_h[i][j], i = key index, j = value index
 *           (the GPU arena layout of shaders/gdn.comp:2), updated in place.
 *   out   : f32 out[t*out_tok_stride + h*S + j] = (S_h^T q)_j / sqrt(S)
 * Requires S == 128, nv % nk == 0.
 * Replaces the gdn / gdn_p dispatches, src/vk/mod.rs:805-806 and the per-token MTP-verify loop
 * 797-801 (kernels/src/lib.rs:252-331; CPU cpu.rs:216-232). */
int it_gdn_step(const float* co, int co_tok_stride, const float* beta_raw, const float* alpha_raw,
                int ba_tok_stride, const float* dt, const float* a, float* state, float* out,
                int out_tok_stride, int nt, int nv, int nk, int S, void* stream);

/* A GDN decode layer in one launch: it_gdn_conv_l2norm (nnorm = 2*nk) followed by it_gdn_step,
 * for 1 <= nt <= 4 tokens, without the conv output ever reaching memory.
 *   x, x_tok_stride, w, K : as for it_gdn_conv (cd = (2*nk + nv)*S); x and w 16-byte aligned,
 *                           stride % 4 == 0
 *   conv_state_in         : f32 [(K-1)][cd], the conv state before token 0 (read only)
 *   conv_state_out        : f32 [(K-1)][cd], receives the conv state after token nt-1; it must not
 *                           overlap conv_state_in (every workgroup reads the old state while others
 *                           write the new one: callers alternate two buffers)
 *   the rest              : as for it_gdn_step (state updated in place), eps as for the L2 norm.
 * Replaces the conv, rmsnorm mode 2 and gdn dispatch triple, src/vk/mod.rs:803-806 (cpu.rs:201-232). */
int it_gdn_decode_fused(const float* x, int x_tok_stride, const float* w, int K, const float* conv_state_in,
                        float* conv_state_out, const float* beta_raw, const float* alpha_raw, int ba_tok_stride,
                        const float* dt, const float* a, float* state, float* out, int out_tok_stride, int nt,
                        int nv, int nk, int S, float eps, void* stream);

/* it_gdn_decode_fused for an MTP verify batch, plus the checkpoints of both states after token
 * ck_after (0 <= ck_after < nt), written from registers: ck_state [nv][S][S] (the recurrent state,
 * as it_gdn_step_ckpt) and ck_conv [(K-1)][cd] (the conv state, as it_gdn_conv_l2norm_ckpt). Neither
 * may overlap the state it snapshots or the other buffers.
 * Replaces the verify loop's conv / rmsnorm / gdn dispatches and checkpoint copies,
 * src/vk/mod.rs:790-806 (mtp.rs:227-234). */
int it_gdn_decode_fused_ckpt(const float* x, int x_tok_stride, const float* w, int K, const float* conv_state_in,
                             float* conv_state_out, const float* beta_raw, const float* alpha_raw,
                             int ba_tok_stride, const float* dt, const float* a, float* state, float* out,
                             int out_tok_stride, int nt, int nv, int nk, int S, float eps, float* ck_state,
                             float* ck_conv, int ck_after, void* stream);

/* The GDN output's gated RMSNorm, per (token t, V head h) row of S = 128:
 *   out[t*out_tok_stride + h*S + j] = o_j / sqrt(mean_j(o^2) + eps) * w[j] * silu(z[t*z_tok_stride + h*S + j])
 * with o the row o[t*o_tok_stride + h*S ...] and w [S] (ssm_norm, shared by the heads). out may be
 * o itself (in place, like the reference) or a buffer that does not overlap it.
 * Replaces rmsnorm mode 1, src/vk/mod.rs:808 (kernels/src/lib.rs:207-229; cpu.rs:234-238). */
int it_gdn_gated_rmsnorm(const float* o, int o_tok_stride, const float* z, int z_tok_stride, const float* w,
                         float eps, float* out, int out_tok_stride, int nv, int S, int nt, void* stream);

/* it_gdn_step with the gated RMSNorm fused into the output write: one workgroup per V head holds
 * the head's whole state, so each token's output row is complete before it is stored.
 *   z, norm_w, eps: as for it_gdn_gated_rmsnorm (z 16-byte aligned, z_tok_stride a multiple of 4);
 *          z == NULL writes the plain recurrence output (same values as it_gdn_step).
 *   ck_state, ck_after: the optional MTP verify checkpoint as in it_gdn_step_ckpt (NULL = none).
 * Replaces the gdn dispatch plus rmsnorm mode 1, src/vk/mod.rs:805-808 (cpu.rs:216-238). */
int it_gdn_step_gated(const float* co, int co_tok_stride, const float* beta_raw, const float* alpha_raw,
                      int ba_tok_stride, const float* dt, const float* a, float* state, float* out,
                      int out_tok_stride, int nt, int nv, int nk, int S, const float* z, int z_tok_stride,
                      const float* norm_w, float eps, float* ck_state, int ck_after, void* stream);

/* ------------------------------------------------------------------------------------------------
 * MTP verify checkpoint and rollback of the recurrent state.
 * The reference runs a verify batch (the accepted token x and the draft d) one token at a time and
 * copies the conv and SSM states after token 0 into checkpoint buffers (src/vk/mod.rs:790-801); a
 * rejected draft copies them back (mtp_reject, src/vk/mod.rs:1018-1025; CPU: mtp.rs:227-234).
 * Here the kernels that already hold the state for the whole token run write the checkpoint from
 * registers after token ck_after (0 <= ck_after < nt), without a second pass over the state.
 * ck_state has the layout of the state it snapshots and must not overlap it.
 * ---------------------------------------------------------------------------------------------- */

/* it_gdn_conv, plus ck_state[i*cd + ch] = the conv state after token ck_after. */
int it_gdn_conv_ckpt(const float* x, int x_tok_stride, const float* w, float* state, float* out,
                     int out_tok_stride, int cd, int nt, int K, float* ck_state, int ck_after, void* stream);

/* it_gdn_conv_l2norm, plus the conv-state checkpoint after token ck_after. */
int it_gdn_conv_l2norm_ckpt(const float* x, int x_tok_stride, const float* w, float* state, float* out,
                            int out_tok_stride, int cd, int nt, int K, int nnorm, float eps, float* ck_state,
                            int ck_after, void* stream);

/* it_gdn_step, plus ck_state[h][i][j] = the SSM state after token ck_after (16-byte aligned). */
int it_gdn_step_ckpt(const float* co, int co_tok_stride, const float* beta_raw, const float* alpha_raw,
                     int ba_tok_stride, const float* dt, const float* a, float* state, float* out,
                     int out_tok_stride, int nt, int nv, int nk, int S, float* ck_state, int ck_after,
                     void* stream);

/* Rollback after a rejected draft: conv_state <- ck_conv (conv_words floats) and ssm <- ck_ssm
 * (ssm_words floats), both in one copy kernel on the stream (either count may be 0; no buffer may
 * overlap another). */
int it_gdn_rollback(const float* ck_conv, float* conv_state, size_t conv_words, const float* ck_ssm, float* ssm,
                    size_t ssm_words, void* stream);

/* Same contract and result as it_gdn_step over nt tokens, computed with the chunk-64 WY/UT form of
 * the gated delta rule on f16 MFMA with f32 state and accumulation (a new algorithm: the reference
 * runs the recurrence token-sequentially, kernels/src/lib.rs:285-331). Scratch as returned by
 * it_gdn_chunked_scratch_bytes. The q and k heads must be L2-normalised, as the layer's rmsnorm
 * mode 2 leaves them before the recurrence (cpu.rs:214): the chunk operands are kept as f16, which
 * assumes |k| <= 1 (it_gdn_step has no such bound). */
size_t it_gdn_chunked_scratch_bytes(int nt, int nv, int S);
int it_gdn_chunked(const float* co, int co_tok_stride, const float* beta_raw, const float* alpha_raw,
                   int ba_tok_stride, const float* dt, const float* a, float* state, float* out,
                   int out_tok_stride, int nt, int nv, int nk, int S, void* scratch,
                   size_t scratch_bytes, void* stream);

/* The GDN layer over a prompt chunk in one call: replaces the conv (src/vk/mod.rs:803), rmsnorm
 * mode 2 on the q/k heads (804) and gdn_p (806) dispatches of a prefill chunk. Conv + SiLU + q/k
 * L2 norm (as it_gdn_conv_l2norm with nnorm = 2*nk), its output kept in `scratch` as f16 (the
 * "f16 activations" of the chunked-prefill benchmark: half the bytes for the conv's write and the
 * scan's read; at 8192 tokens the outputs are within ~1.2e-4 and the final state within ~8.5e-4
 * of the f32 token-sequential reference, against ~8e-5 / ~4.4e-4 from an f32 conv output),
 * then the chunk-64 scan of it_gdn_chunked. x [nt][x_tok_stride] f32 with cd = (2*nk+nv)*S
 * channels; w, conv_state, beta_raw, alpha_raw, dt, a, state and out as it_gdn_conv and
 * it_gdn_chunked (S = 128); conv_state and state are updated in place. scratch: 16-byte aligned,
 * it_gdn_prefill_scratch_bytes(nt, nv, nk, S) bytes. */
size_t it_gdn_prefill_scratch_bytes(int nt, int nv, int nk, int S);
int it_gdn_prefill(const float* x, int x_tok_stride, const float* conv_w, int K, float* conv_state,
                   const float* beta_raw, const float* alpha_raw, int ba_tok_stride, const float* dt,
                   const float* a, float* state, float* out, int out_tok_stride, int nt, int nv, int nk, int S,
                   float eps, void* scratch, size_t scratch_bytes, void* stream);

/* ------------------------------------------------------------------------------------------------
 * Reference-shaped dispatch policy (pure host functions, no device access).
 * ---------------------------------------------------------------------------------------------- */

/* 64*heads*max(ctx,260) (src/vk/mod.rs:138): the arena's scratch words for a 64-token batch. An
 * arena for larger chunks holds it_attention_dispatch_room(ctx, heads, ubatch) words, as the
 * reference's scr slot does (src/vk/mod.rs:546). */
size_t it_attention_scratch_words(size_t ctx, size_t heads);
/* ceil(nt/64)*64*heads*max(ctx,260), nt in 1..=512 (src/vk/mod.rs:148-150); 0 if nt is invalid. */
size_t it_attention_dispatch_room(size_t ctx, size_t heads, size_t nt);
/* Keys per split the reference would choose: 64 doubled (at most to 1024) until
 * nt*nh*ceil((pos0+nt)/C)*260 <= room (src/vk/mod.rs:714-716); -1 if even 1024 does not fit. */
int it_attention_chunk(uint32_t nt, uint32_t nh, uint32_t pos0, size_t room);
/* The prompt split of src/vk/mod.rs:130-134 (prefill_chunks): consecutive ranges of at most `batch`
 * tokens (batch 64, 128, 256 or 512) covering 0..len, where a range longer than 64 whose length
 * leaves a tail of 1..21 tokens past a multiple of 64 gives that tail to the next range (no token
 * is dropped or repeated). Range i is starts[i] .. starts[i]+lens[i]. Writes at most cap ranges and
 * returns the number of ranges (which may exceed cap), or -1 if batch is not 64/128/256/512. */
long it_prefill_chunks(size_t len, size_t batch, size_t* starts, size_t* lens, size_t cap);
/* Geometry check of src/vk/mod.rs:207-220 restricted to the attention/GDN fields; 0 = supported. */
int it_validate_geometry(int ctx_len, int head_dim, int n_head, int n_head_kv, int ssm_state,
                         int ssm_groups, int ssm_vheads, int ssm_inner, int conv_k);

/* Measurement only, no counterpart in the reference: the device's sustained f16 matrix-core
 * rate. wgs workgroups of 256 threads; each of their waves issues 4 * iters independent
 * 32x32x16 f16 MFMAs (32768 flops each) and touches no memory besides one float per thread
 * written to out (wgs * 256 floats). Rate = wgs * 4 * 4 * iters * 32768 / elapsed time. */
int it_calib_mfma_f16(int wgs, int iters, float* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* IT_ATTN_H */
