// Launch functions shared between the kernel files and the C ABI layer (api.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "rec_index.h"

namespace it {

hipError_t launch_kv_append(const float* k, const float* v, int sts, uint16_t* kc, uint16_t* vc, int pos0, int nt,
                            int kvd, int rtz, hipStream_t st);
hipError_t launch_attn_prep(float* q, int qts, const float* k, const float* v, int kts, const float* qw,
                            const float* kw, float eps, uint16_t* kc, uint16_t* vc, int pos0, int hd, int nh, int nkv,
                            int nt, int n_rot, float tsc, const int* sec, int rtz, hipStream_t st,
                            uint16_t* q16 = nullptr, int q16ts = 0, float q16s = 0.f);
hipError_t launch_attn_prep_f32kv(float* q, int qts, const float* k, const float* v, int kts, const float* qw,
                                  const float* kw, float eps, float* kc, float* vc, int pos0, int row0, int hd, int nh,
                                  int nkv, int nt, int n_rot, float tsc, const int* sec, hipStream_t st);
hipError_t launch_attn_f32kv(const float* q, int qts, const float* kc, const float* vc, int kvd, int pos0, int nh,
                             int nkv, int nt, float scale, float* out, int ots, float* part, int chunk, hipStream_t st);
// pieces: the split records in decode.hip's piece layout (for the wave merge only: piece_records());
// false: the 260-word f32 records {m, l, 0, 0, o[256]} that it_attn_partials / it_attn_combine
// exchange
bool piece_records(int pos0, int nt, int nh, int chunk);
hipError_t launch_attn_partials(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                                int nh, int nkv, int nt, float scale, float* part, int chunk, hipStream_t st,
                                bool pieces = false);
hipError_t launch_attn_combine(const float* q, int qts, const float* part, int pos0, int nh, int nt, int chunk,
                               float* out, int ots, hipStream_t st, bool pieces = false);
// Key-split flash records in the compact form: {m, l, k, 0} + 256 int16 (O in units of k).
constexpr int FLASH_REC = idx::FLASH_REC;
// log2(e): the flash kernel works in log2 units (its q operand is q * scale * LOG2E)
constexpr float LOG2E = 1.4426950408889634f;
hipError_t launch_attn_combine_q16(const float* q, int qts, const float* part, int pos0, int nh, int nt, int chunk,
                                   float* out, int ots, hipStream_t st);
hipError_t launch_attn_splitk(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                              int nh, int nkv, int nt, float scale, float* out, int ots, float* part, int chunk,
                              hipStream_t st);
// Decode attention in one launch through a mailbox (see decode.hip). Returns hipSuccess with
// *launched = false, having enqueued nothing, when the geometry does not qualify (splits of 64
// keys, at most 256 splits, at most 8 query rows per KV head, a wave per (row, 16-dim block) merge
// unit, mailbox_bytes(pos0 + nt, nt, nh) bytes, the whole grid co-resident on the device); with
// dry_run, only reports whether it would launch.
size_t mailbox_bytes(long ctx, int nt, int nh);
// mailbox header: word 0 the poison flag (0 = clear), word 1 this value once initialised
constexpr uint32_t MAILBOX_MAGIC = 0x4D424F58u;
hipError_t launch_attn_decode_mailbox(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd,
                                      int pos0, int nh, int nkv, int nt, float scale, float* out, int ots, float* mb,
                                      size_t mbb, hipStream_t st, bool* launched, bool dry_run = false);
// report: device address of a host-visible word the fill clears and a merge that finds the
// mailbox poisoned sets (null: none)
hipError_t launch_mailbox_fill(void* mb, size_t bytes, uint32_t* report, hipStream_t st);
// q16 (optional): the q operand pre-converted, q16[t * q16ts + h * 256 + d] = f16(q * scale * LOG2E)
hipError_t launch_attn_flash(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                             int nh, int nkv, int nt, float scale, float* out, int ots, hipStream_t st,
                             const uint16_t* q16 = nullptr, int q16ts = 0);

int flash_split_chunk(int pos0, int nt, int nh, int nkv);
hipError_t launch_attn_flash_split(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0,
                                   int nh, int nkv, int nt, float scale, float* out, int ots, float* part, int chunk,
                                   hipStream_t st, bool f32rec = false, const uint16_t* q16 = nullptr,
                                   int q16ts = 0);

// ck / ck_after: optional checkpoint of the state after token ck_after (null = none).
hipError_t launch_gdn_conv(const float* x, int xts, const float* w, float* state, float* out, int ots, int cd, int nt,
                           int K, float* ck, int ck_after, hipStream_t st);
// OutT float or _Float16 (the conv output as f16 for the one-call GDN prefill)
template <typename OutT>
hipError_t launch_gdn_conv_l2(const float* x, int xts, const float* w, float* state, OutT* out, int ots, int cd,
                              int nt, int K, int nnorm, float eps, float* ck, int ck_after, hipStream_t st);
hipError_t launch_l2norm(float* x, int ts, int nheads, int d, int nt, float eps, hipStream_t st);
hipError_t launch_gdn_decode_fused(const float* x, int xts, const float* cw, int K, const float* cst_in, float* cst_out,
                                   const float* br, const float* ar, int bts, const float* dt, const float* a,
                                   float* state, float* out, int ots, int nt, int nv, int nk, float eps,
                                   float* ck_state, float* ck_conv, int ck_after, hipStream_t st);
hipError_t launch_gdn_step(const float* co, int cts, const float* br, const float* ar, int bts, const float* dt,
                           const float* a, float* state, float* out, int ots, int nt, int nv, int nk, float* ck,
                           int ck_after, hipStream_t st);
hipError_t launch_gdn_step_head(const float* co, int cts, const float* br, const float* ar, int bts, const float* dt,
                                const float* a, float* state, float* out, int ots, int nt, int nv, int nk,
                                const float* z, int zts, const float* nw, float eps, float* ck, int ck_after,
                                hipStream_t st);
hipError_t launch_gdn_gated_norm(const float* o, int ots, const float* z, int zts, const float* w, float eps,
                                 float* out, int outs, int nv, int nt, hipStream_t st);
size_t gdn_chunked_scratch_bytes(int nt, int nv, int S, bool f16_conv);
// CoT float (it_gdn_chunked) or _Float16 (the conv output of the one-call GDN prefill)
template <typename CoT>
hipError_t launch_gdn_chunked(const CoT* co, int cts, const float* br, const float* ar, int bts, const float* dt,
                              const float* a, float* state, float* out, int ots, int nt, int nv, int nk, void* scratch,
                              hipStream_t st);

// f16 matrix-core rate probe: wgs workgroups of 4 waves, each wave 4 x iters 32x32x16 MFMAs;
// out receives wgs * 256 floats.
hipError_t launch_mfma_peak(int wgs, int iters, float* out, hipStream_t st);

// conv <- ck_conv (nc floats) and ssm <- ck_ssm (ns floats) in one launch.
hipError_t launch_gdn_rollback(const float* ck_conv, float* conv, size_t nc, const float* ck_ssm, float* ssm,
                               size_t ns, hipStream_t st);

}  // namespace it
