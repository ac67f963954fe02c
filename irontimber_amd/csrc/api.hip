// C ABI of the hot path (declared in include/it_attn.h): host-side validation, dispatch policy and
// kernel launches. Validation runs before any device work, like the reference's fail-closed
// checks (src/vk/mod.rs:179-220); runtime errors come back as nonzero codes with a thread-local
// message instead of the reference's panics.
#include <mutex>
#include <unordered_map>
#include <utility>
#include <string>
#include <cstdio>
#include <cstdarg>
#include "../../include/it_attn.h"
#include "internal.h"

namespace {

thread_local std::string g_err;

int fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return -1;
}
int check(hipError_t e, const char* what) {
    if (e != hipSuccess) return fail("%s: %s", what, hipGetErrorString(e));
    g_err.clear();
    return 0;
}
bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

constexpr int HD = 256;
constexpr size_t PART_WORDS = it::idx::PART;
constexpr int KERNEL_AUTO = 0, KERNEL_SPLITK = 1, KERNEL_FLASH = 2, KERNEL_FLASH_F32 = 3;
constexpr size_t AUTO_SCRATCH_CAP = size_t(256) << 20;   // keep automatic split-K scratch under 256 MiB

// Keys per split for the split-K kernel when the caller leaves it to us: one 64-key tile per
// workgroup (ctx 8192 -> 128 splits per KV head, 256 workgroups for two KV heads), doubled only
// when the partial records would outgrow the scratch cap. Decode and 2-token calls below 2048 keys
// take 32-key splits (the tile's second half masked): with 64-key splits those leave most CUs idle
// (ctx 1024: 32 workgroups); same box, 32 against 64 keys, ctx 256 / 512 / 1024 / 1984: 5.76 /
// 5.86 / 6.16 / 6.36 against 5.89 / 6.13 / 6.53 / 6.60 us, 2 tokens at 512 / 1024: 6.08 / 6.33
// against 6.16 / 6.65 us; 4-token calls measured better with 64 keys at 768-2048 keys. From 2048
// keys, and wherever the one-launch mailbox form can launch (it uses 64-key splits; the two forms
// stay bit-equal), the split stays at 64: the mailbox needs at most 8 query rows per KV head and at
// most 4 merge units (row, 16-dim block) per workgroup. The f32-KV kernel's tiles cover whole
// splits, so it asks for 64-key splits (short_splits = false).
int auto_chunk(int pos0, int nt, int nh, int nkv, bool short_splits = true) {
    const size_t total = (size_t)pos0 + nt;
    const long R = (long)nt * (nh / nkv);                          // query rows per KV head
    const long wgs64 = (long)((total + 63) / 64) * nkv * ((R + 7) / 8);
    const bool mailbox_possible = R <= 8 && (long)nt * nh * 16 <= 4 * wgs64;
    int c = short_splits && nt <= 2 && total < 2048 && !mailbox_possible ? 32 : 64;
    while (c < (1 << 20) && (size_t)nt * nh * ((total + c - 1) / c) * PART_WORDS * 4 > AUTO_SCRATCH_CAP) c *= 2;
    return c;
}
int auto_kernel(int nt) { return nt >= 16 ? KERNEL_FLASH : KERNEL_SPLITK; }

// Keys per split of the flash kernel: the caller's chunk, or the library's choice when 0; 0 back
// means one pass over all keys (no scratch).
int flash_chunk(int pos0, int nt, int nh, int nkv, int chunk) {
    const int c = chunk > 0 ? chunk : it::flash_split_chunk(pos0, nt, nh, nkv);
    return (c > 0 && c < pos0 + nt) ? c : 0;
}

size_t splitk_scratch(int pos0, int nt, int nh, int chunk) {
    const size_t smax = (size_t)it::idx::split_count((long)pos0 + nt, chunk);
    return (size_t)nt * nh * smax * PART_WORDS * sizeof(float);
}

// Scratch of the flash kernel's key-split records: it::FLASH_REC words (16-byte header and O as
// int16) per (token, head, split), half the split-K kernel's 260-word f32 records.
// With f32 records (kernel 3) the records are the split-K kernel's 260 words instead.
size_t flash_scratch(int pos0, int nt, int nh, int chunk, bool f32rec = false) {
    const size_t smax = (size_t)it::idx::split_count((long)pos0 + nt, chunk);
    return (size_t)nt * nh * smax * (f32rec ? PART_WORDS : (size_t)it::FLASH_REC) * sizeof(float);
}

// Kernel and keys per split for an automatic call that must fit `budget` bytes of scratch. The
// library's preferred split is kept when it fits; otherwise the split doubles until the records
// fit, which is the reference's rule for its fixed arena (src/vk/mod.rs:714-716: C doubles from 64
// while nt*nh*ceil((pos0+nt)/C)*260 words exceed the room). The flash kernel ends at one pass over
// all keys, which needs no scratch, so it always has a plan; the split-K kernel (nt < 16) can run
// out of doublings only when even one record per (token, head) exceeds the budget. A chunk of 0
// from the flash plan means the one-pass form. Returns false if nothing fits.
struct AttnPlan { int kernel, chunk; size_t bytes; };
bool plan_attn(int pos0, int nt, int nh, int nkv, int kernel, size_t budget, AttnPlan& p) {
    const long total = (long)pos0 + nt;
    if (kernel == KERNEL_AUTO) kernel = auto_kernel(nt);
    p.kernel = kernel;
    if (kernel == KERNEL_FLASH || kernel == KERNEL_FLASH_F32) {
        const bool f32 = kernel == KERNEL_FLASH_F32;
        int c = flash_chunk(pos0, nt, nh, nkv, 0);
        while (c && flash_scratch(pos0, nt, nh, c, f32) > budget) c = (2L * c >= total) ? 0 : 2 * c;
        p.chunk = c;
        p.bytes = c ? flash_scratch(pos0, nt, nh, c, f32) : 0;
        return true;
    }
    int c = auto_chunk(pos0, nt, nh, nkv);
    while (splitk_scratch(pos0, nt, nh, c) > budget && c < total) c *= 2;
    p.chunk = c;
    p.bytes = splitk_scratch(pos0, nt, nh, c);
    return p.bytes <= budget;
}

// Keys per split for the f32-KV (MTP head) attention that must fit `budget` bytes of scratch: the
// library's preferred split when it fits, else the split doubles until the 260-word records fit
// (the reference's rule for this call, src/vk/mod.rs:730-733). The kernel walks any number of
// 64-key tiles per split, so the doubling may go on past the reference's 1024 keys up to one split
// over every key. If even one record per (token, head) does not fit, chunk 0: one pass that
// writes the output directly and needs no scratch (the reference falls back to its whole-context
// `attn` kernel there, src/vk/mod.rs:740). Always succeeds.
struct F32kvPlan { int chunk; size_t bytes; };
// The f32-KV kernel's preferred split. Calls of one block of query rows (decode, verify: up to 32
// rows per KV head) keep one 64-key tile per split. Calls with several row blocks (the 64-token
// catch-up) read each K/V tile once per block and hold one workgroup per CU (133 KB of LDS), so
// their time goes as the number of rounds of workgroups over the CUs times the tiles a workgroup
// walks: the split (a multiple of 64 keys) minimises rounds x (tiles + 1), the + 1 standing for a
// workgroup's fixed cost (q rows, first tile, records), ties going to the longer split (fewer
// records). A fixed 256-key split gave 99 us for 64 tokens at slot 4096 (544 workgroups: 3 rounds
// of 4 tiles); 320 / 384 / 512 keys gave 81 / 91 / 114 us (2 rounds of 5 / 6 / 8 tiles).
constexpr int F32KV_CUS = 256;   // MI355X compute units
int f32kv_pref_chunk(int pos0, int nt, int nh, int nkv) {
    const int G = nh / nkv;
    if ((long)nt * G <= 32) return auto_chunk(pos0, nt, nh, nkv, false);
    const long total = (long)pos0 + nt;
    const long blocks = ((long)nt * G + 31) / 32;   // 32-row blocks of the multi-block kernel
    int best = 64;
    long best_cost = -1;
    for (long c = 64;; c += 64) {
        const long wgs = (total + c - 1) / c * nkv * blocks;
        const long cost = (wgs + F32KV_CUS - 1) / F32KV_CUS * (c / 64 + 1);
        if (best_cost < 0 || cost <= best_cost) {
            best_cost = cost;
            best = (int)c;
        }
        if (c >= total) break;
    }
    return best;
}
F32kvPlan plan_f32kv(int pos0, int nt, int nh, int nkv, size_t budget) {
    const long total = (long)pos0 + nt;
    int c = f32kv_pref_chunk(pos0, nt, nh, nkv);
    while (splitk_scratch(pos0, nt, nh, c) > budget && c < total) c *= 2;
    if (splitk_scratch(pos0, nt, nh, c) > budget) return {0, 0};
    return {c, splitk_scratch(pos0, nt, nh, c)};
}

int validate_attn(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0, int hd, int nh,
                  int nkv, int nt, const float* out, int ots) {
    if (hd != HD) return fail("it_attn_f16: head_dim %d unsupported (the f16 KV path requires 256)", hd);
    if (nh <= 0 || nkv <= 0 || nh % nkv != 0) return fail("it_attn_f16: n_head %d / n_head_kv %d invalid", nh, nkv);
    if (kvd != nkv * hd) return fail("it_attn_f16: kvd %d != n_head_kv*head_dim %d", kvd, nkv * hd);
    if (nt <= 0 || pos0 < 0) return fail("it_attn_f16: nt %d / pos0 %d invalid", nt, pos0);
    if ((long)pos0 + nt > (1L << 22)) return fail("it_attn_f16: context %ld too long", (long)pos0 + nt);
    if (!q || !kc || !vc || !out) return fail("it_attn_f16: null buffer");
    if (!aligned16(q) || !aligned16(kc) || !aligned16(vc) || !aligned16(out))
        return fail("it_attn_f16: q/kc/vc/out must be 16-byte aligned");
    if (qts % 4 != 0 || ots % 4 != 0) return fail("it_attn_f16: token strides must be multiples of 4");
    if (nt > 1 && (qts < 2 * nh * hd || ots < nh * hd)) return fail("it_attn_f16: token strides overlap rows");
    return 0;
}

// ---- the no-allocation variant of it_attn_f16 ------------------------------------------------
// Its split-K partial records live in this file-scope device array instead of a caller buffer.
// Every GPU the library runs on holds its own copy (IT_NOALLOC_SCRATCH_BYTES) until the process
// ends. In host code `scratch` names a host-side stand-in, not the device copy: the device address
// comes from hipGetSymbolAddress, once per device with that device current, and only that address
// is passed to kernels.
static __device__ __align__(256) unsigned char scratch[IT_NOALLOC_SCRATCH_BYTES];

constexpr int NOALLOC_MAX_DEV = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[NOALLOC_MAX_DEV] = {};

// Device address of the current device's `scratch` (looked up on the first call per device).
int noalloc_scratch(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail("it_attn_f16_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= NOALLOC_MAX_DEV) return fail("it_attn_f16_noalloc: device %d beyond %d", dev, NOALLOC_MAX_DEV);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail("it_attn_f16_noalloc: hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return 0;
}

// Host-visible report words of the mailboxes this process initialised (one pinned, coherent word
// each, kept until the process ends): a merge that finds its mailbox poisoned sets the word, and
// it_attn_f16_mailbox checks it without touching the device.
std::mutex g_report_mu;
std::unordered_map<const void*, std::pair<volatile uint32_t*, uint32_t*>> g_report;

int mailbox_report(const void* mailbox, bool create, volatile uint32_t** host, uint32_t** dev) {
    std::lock_guard<std::mutex> lk(g_report_mu);
    auto it = g_report.find(mailbox);
    if (it == g_report.end()) {
        if (!create) { *host = nullptr; if (dev) *dev = nullptr; return 0; }
        void* h = nullptr;
        hipError_t e = hipHostMalloc(&h, 64, hipHostMallocCoherent | hipHostMallocMapped | hipHostMallocPortable);
        if (e != hipSuccess) return fail("it_attn_mailbox_init: hipHostMalloc: %s", hipGetErrorString(e));
        void* d = nullptr;
        e = hipHostGetDevicePointer(&d, h, 0);
        if (e != hipSuccess) return fail("it_attn_mailbox_init: hipHostGetDevicePointer: %s", hipGetErrorString(e));
        *(volatile uint32_t*)h = 0;
        it = g_report.emplace(mailbox, std::make_pair((volatile uint32_t*)h, (uint32_t*)d)).first;
    }
    *host = it->second.first;
    if (dev) *dev = it->second.second;
    return 0;
}

}  // namespace

extern "C" {

const char* it_last_error(void) { return g_err.c_str(); }
int it_abi_version(void) { return 1; }

int it_kv_append_f16(const float* k, const float* v, int src_tok_stride, uint16_t* kc, uint16_t* vc, int pos0, int nt,
                     int kvd, int round_mode, void* stream) {
    if (nt < 0 || pos0 < 0 || kvd <= 0 || kvd % 4 != 0) return fail("it_kv_append_f16: bad geometry nt=%d pos0=%d kvd=%d", nt, pos0, kvd);
    if (round_mode != 0 && round_mode != 1) return fail("it_kv_append_f16: round_mode must be 0 (RNE) or 1 (RTZ)");
    if (nt > 1 && src_tok_stride < kvd) return fail("it_kv_append_f16: source stride %d < kvd %d", src_tok_stride, kvd);
    if (src_tok_stride % 4 != 0) return fail("it_kv_append_f16: source stride must be a multiple of 4");
    if (!k || !v || !kc || !vc || !aligned16(k) || !aligned16(v) || !aligned16(kc) || !aligned16(vc))
        return fail("it_kv_append_f16: buffers must be non-null and 16-byte aligned");
    return check(it::launch_kv_append(k, v, src_tok_stride, kc, vc, pos0, nt, kvd, round_mode, (hipStream_t)stream),
                 "it_kv_append_f16");
}

static int validate_prep(const char* who, const float* q, int qts, const float* k, const float* v, int kts,
                         const float* q_norm, const float* k_norm, float eps, const void* kc, const void* vc, int kvd,
                         int pos0, int hd, int nh, int nkv, int nt, int n_rot, float theta_scale, int sec0, int sec1,
                         int sec2, int sec3) {
    if (hd != 128 && hd != 256) return fail("%s: head_dim %d unsupported (128 or 256)", who, hd);
    if (nh <= 0 || nkv <= 0 || nh % nkv != 0) return fail("%s: n_head %d / n_head_kv %d invalid", who, nh, nkv);
    if (kvd != nkv * hd) return fail("%s: kvd %d != n_head_kv*head_dim %d", who, kvd, nkv * hd);
    if (nt < 0 || pos0 < 0 || (long)pos0 + nt > (1L << 22)) return fail("%s: nt %d / pos0 %d invalid", who, nt, pos0);
    const int per_lane = hd / 64;
    if (n_rot < 0 || n_rot > hd || n_rot % (2 * per_lane) != 0)
        return fail("%s: n_rot %d must be in [0, %d] and a multiple of %d", who, n_rot, hd, 2 * per_lane);
    if (sec0 < 0 || sec1 < 0 || sec2 < 0 || sec3 < 0) return fail("%s: rope sections must be >= 0", who);
    if (!(theta_scale > 0.0f) || !(theta_scale <= 1.0f)) return fail("%s: theta_scale %g must be in (0, 1]", who, theta_scale);
    if (!(eps >= 0.0f)) return fail("%s: eps must be >= 0", who);
    if (!q || !k || !v || !kc || !vc) return fail("%s: null buffer", who);
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(kc) || !aligned16(vc) ||
        (q_norm && !aligned16(q_norm)) || (k_norm && !aligned16(k_norm)))
        return fail("%s: buffers must be 16-byte aligned", who);
    if (qts % 4 != 0 || kts % 4 != 0) return fail("%s: token strides must be multiples of 4", who);
    if (nt > 1 && (qts < 2 * nh * hd || kts < kvd)) return fail("%s: token strides overlap rows", who);
    return 0;
}

int it_attn_prep_f16(float* q, int qts, const float* k, const float* v, int kts, const float* q_norm,
                     const float* k_norm, float eps, uint16_t* kc, uint16_t* vc, int kvd, int pos0, int hd, int nh,
                     int nkv, int nt, int n_rot, float theta_scale, int sec0, int sec1, int sec2, int sec3,
                     int round_mode, void* stream) {
    const char* who = "it_attn_prep_f16";
    if (validate_prep(who, q, qts, k, v, kts, q_norm, k_norm, eps, kc, vc, kvd, pos0, hd, nh, nkv, nt, n_rot,
                      theta_scale, sec0, sec1, sec2, sec3))
        return -1;
    if (round_mode != 0 && round_mode != 1) return fail("%s: round_mode must be 0 (RNE) or 1 (RTZ)", who);
    if (nt == 0) { g_err.clear(); return 0; }
    const int sec[4] = {sec0, sec1, sec2, sec3};
    return check(it::launch_attn_prep(q, qts, k, v, kts, q_norm, k_norm, eps, kc, vc, pos0, hd, nh, nkv, nt, n_rot,
                                      theta_scale, sec, round_mode, (hipStream_t)stream),
                 who);
}

int it_attn_prep_f16_q16(float* q, int qts, const float* k, const float* v, int kts, const float* q_norm,
                         const float* k_norm, float eps, uint16_t* kc, uint16_t* vc, int kvd, int pos0, int hd, int nh,
                         int nkv, int nt, int n_rot, float theta_scale, int sec0, int sec1, int sec2, int sec3,
                         int round_mode, uint16_t* q16, int q16ts, float scale, void* stream) {
    const char* who = "it_attn_prep_f16_q16";
    if (validate_prep(who, q, qts, k, v, kts, q_norm, k_norm, eps, kc, vc, kvd, pos0, hd, nh, nkv, nt, n_rot,
                      theta_scale, sec0, sec1, sec2, sec3))
        return -1;
    if (round_mode != 0 && round_mode != 1) return fail("%s: round_mode must be 0 (RNE) or 1 (RTZ)", who);
    if (!q16) return fail("%s: null q16", who);
    if (!aligned16(q16) || q16ts % 8 != 0) return fail("%s: q16 must be 16-byte aligned, its token stride a multiple of 8", who);
    if (nt > 1 && q16ts < nh * hd) return fail("%s: q16 token stride %d overlaps rows", who, q16ts);
    if (!(scale > 0.0f) || !(scale < 1e30f)) return fail("%s: scale %g invalid", who, scale);
    if (nt == 0) { g_err.clear(); return 0; }
    const int sec[4] = {sec0, sec1, sec2, sec3};
    // the flash kernel's own conversion: f16(q * (scale * LOG2E)), the product in f32
    const float q16s = scale * it::LOG2E;
    return check(it::launch_attn_prep(q, qts, k, v, kts, q_norm, k_norm, eps, kc, vc, pos0, hd, nh, nkv, nt, n_rot,
                                      theta_scale, sec, round_mode, (hipStream_t)stream, q16, q16ts, q16s),
                 who);
}

int it_attn_prep_f32kv(float* q, int qts, const float* k, const float* v, int kts, const float* q_norm,
                       const float* k_norm, float eps, float* kc, float* vc, int kvd, int pos0, int row0, int hd,
                       int nh, int nkv, int nt, int n_rot, float theta_scale, int sec0, int sec1, int sec2, int sec3,
                       void* stream) {
    const char* who = "it_attn_prep_f32kv";
    if (validate_prep(who, q, qts, k, v, kts, q_norm, k_norm, eps, kc, vc, kvd, pos0, hd, nh, nkv, nt, n_rot,
                      theta_scale, sec0, sec1, sec2, sec3))
        return -1;
    if (row0 < 0) return fail("%s: cache row %d invalid", who, row0);
    if (nt == 0) { g_err.clear(); return 0; }
    const int sec[4] = {sec0, sec1, sec2, sec3};
    return check(it::launch_attn_prep_f32kv(q, qts, k, v, kts, q_norm, k_norm, eps, kc, vc, pos0, row0, hd, nh, nkv, nt,
                                            n_rot, theta_scale, sec, (hipStream_t)stream),
                 who);
}

size_t it_attn_f32kv_scratch_bytes(int pos0, int nt, int hd, int nh, int nkv) {
    (void)hd;
    if (nt <= 0 || pos0 < 0 || nh <= 0 || nkv <= 0 || nh % nkv) return 0;
    return splitk_scratch(pos0, nt, nh, f32kv_pref_chunk(pos0, nt, nh, nkv));
}

int it_attn_f32kv_plan(int pos0, int nt, int hd, int nh, int nkv, size_t scratch_bytes, int* chunk, size_t* bytes) {
    if (hd != HD || nt <= 0 || pos0 < 0 || nh <= 0 || nkv <= 0 || nh % nkv || nh / nkv > 16 ||
        (long)pos0 + nt > (1L << 22))
        return fail("it_attn_f32kv_plan: bad geometry");
    const F32kvPlan p = plan_f32kv(pos0, nt, nh, nkv, scratch_bytes);
    if (chunk) *chunk = p.chunk;
    if (bytes) *bytes = p.bytes;
    g_err.clear();
    return 0;
}

int it_attn_f32kv(const float* q, int qts, const float* kc, const float* vc, int kvd, int pos0, int hd, int nh,
                  int nkv, int nt, float scale, float* out, int ots, void* scratch, size_t scratch_bytes,
                  void* stream) {
    const char* who = "it_attn_f32kv";
    if (hd != HD) return fail("%s: head_dim %d unsupported (256)", who, hd);
    if (nh <= 0 || nkv <= 0 || nh % nkv != 0 || nh / nkv > 16)
        return fail("%s: n_head %d / n_head_kv %d invalid (at most 16 q heads per KV head)", who, nh, nkv);
    if (kvd != nkv * hd) return fail("%s: kvd %d != n_head_kv*head_dim %d", who, kvd, nkv * hd);
    if (nt <= 0 || pos0 < 0 || (long)pos0 + nt > (1L << 22)) return fail("%s: nt %d / pos0 %d invalid", who, nt, pos0);
    if (!q || !kc || !vc || !out) return fail("%s: null buffer", who);
    if (!aligned16(q) || !aligned16(kc) || !aligned16(vc) || !aligned16(out))
        return fail("%s: q/kc/vc/out must be 16-byte aligned", who);
    if (qts % 4 != 0 || ots % 4 != 0) return fail("%s: token strides must be multiples of 4", who);
    if (nt > 1 && (qts < 2 * nh * hd || ots < nh * hd)) return fail("%s: token strides overlap rows", who);
    if (scratch && !aligned16(scratch)) return fail("%s: scratch must be 16-byte aligned", who);
    // fit the caller's scratch; no scratch (or too little for one record per row) = one pass
    const F32kvPlan p = plan_f32kv(pos0, nt, nh, nkv, scratch ? scratch_bytes : 0);
    return check(it::launch_attn_f32kv(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, ots, (float*)scratch,
                                       p.chunk, (hipStream_t)stream),
                 who);
}

size_t it_attn_scratch_bytes_ex(int pos0, int nt, int hd, int nh, int nkv, int kernel, int chunk) {
    (void)hd;
    if (nt <= 0 || pos0 < 0 || nh <= 0 || nkv <= 0 || nh % nkv) return 0;
    if (kernel == KERNEL_AUTO) kernel = auto_kernel(nt);
    if (kernel == KERNEL_FLASH || kernel == KERNEL_FLASH_F32) {
        const int c = flash_chunk(pos0, nt, nh, nkv, chunk);
        return c ? flash_scratch(pos0, nt, nh, c, kernel == KERNEL_FLASH_F32) : 0;
    }
    if (kernel != KERNEL_SPLITK) return 0;
    if (chunk <= 0) chunk = auto_chunk(pos0, nt, nh, nkv);
    return splitk_scratch(pos0, nt, nh, chunk);
}
int it_attn_plan(int pos0, int nt, int hd, int nh, int nkv, size_t scratch_bytes, int* kernel, int* chunk,
                 size_t* bytes) {
    if (hd != HD || nt <= 0 || pos0 < 0 || nh <= 0 || nkv <= 0 || nh % nkv || (long)pos0 + nt > (1L << 22))
        return fail("it_attn_plan: bad geometry");
    AttnPlan p;
    const bool ok = plan_attn(pos0, nt, nh, nkv, KERNEL_AUTO, scratch_bytes, p);
    if (kernel) *kernel = p.kernel;
    if (chunk) *chunk = p.chunk;
    if (bytes) *bytes = p.bytes;
    if (!ok) return fail("it_attn_plan: %zu bytes of scratch cannot hold one record per (token, head)", scratch_bytes);
    g_err.clear();
    return 0;
}

size_t it_attn_scratch_bytes(int pos0, int nt, int hd, int nh, int nkv) {
    return it_attn_scratch_bytes_ex(pos0, nt, hd, nh, nkv, KERNEL_AUTO, 0);
}

// it_attn_f16_ex with an optional pre-converted q operand for the flash kernels (q16, see
// it_attn_f16_q16); the split-K (decode, verify) kernels read q as always.
static int attn_f16_impl(const float* q, int qts, const uint16_t* q16, int q16ts, const uint16_t* kc,
                         const uint16_t* vc, int kvd, int pos0, int hd, int nh, int nkv, int nt, float scale,
                         float* out, int ots, void* scratch, size_t scratch_bytes, int kernel, int chunk,
                         void* stream) {
    if (validate_attn(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, out, ots)) return -1;
    if (kernel != KERNEL_AUTO && kernel != KERNEL_SPLITK && kernel != KERNEL_FLASH && kernel != KERNEL_FLASH_F32)
        return fail("it_attn_f16: unknown kernel %d", kernel);
    if (chunk == 0) {
        // automatic split: fit the caller's scratch (the reference's arena rule), never refuse a
        // geometry for which a smaller record set exists
        AttnPlan p;
        if (!plan_attn(pos0, nt, nh, nkv, kernel, scratch ? scratch_bytes : 0, p))
            return fail("it_attn_f16: scratch of %zu bytes cannot hold even one partial record per (token, head) "
                        "(%zu bytes)", scratch_bytes, p.bytes);
        kernel = p.kernel;
        if ((kernel == KERNEL_FLASH || kernel == KERNEL_FLASH_F32) && p.chunk == 0) chunk = 1 << 30;   // one pass
        else chunk = p.chunk;
    }
    if (kernel == KERNEL_AUTO) kernel = auto_kernel(nt);
    hipStream_t st = (hipStream_t)stream;
    if (kernel == KERNEL_FLASH || kernel == KERNEL_FLASH_F32) {
        const bool f32 = kernel == KERNEL_FLASH_F32;
        if (chunk < 0 || chunk % 64 != 0) return fail("it_attn_f16: flash chunk %d must be a multiple of 64", chunk);
        // (chunk is never 0 here: the automatic plan above has replaced it)
        const int c = flash_chunk(pos0, nt, nh, nkv, chunk);
        if (!c)
            return check(it::launch_attn_flash(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, ots, st, q16, q16ts),
                         "it_attn_f16 (flash)");
        const size_t need = flash_scratch(pos0, nt, nh, c, f32);
        if (scratch_bytes < need || !scratch)
            return fail("it_attn_f16: scratch of %zu bytes < %zu required (it_attn_scratch_bytes)", scratch_bytes, need);
        if (!aligned16(scratch)) return fail("it_attn_f16: scratch must be 16-byte aligned");
        return check(it::launch_attn_flash_split(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, ots,
                                                 (float*)scratch, c, st, f32, q16, q16ts),
                     "it_attn_f16 (flash, key splits)");
    }
    if (chunk <= 0) chunk = auto_chunk(pos0, nt, nh, nkv);
    if (chunk % 32 != 0) return fail("it_attn_f16: chunk %d must be a multiple of 32", chunk);
    const size_t need = splitk_scratch(pos0, nt, nh, chunk);
    if (scratch_bytes < need || (need && !scratch))
        return fail("it_attn_f16: scratch of %zu bytes < %zu required (it_attn_scratch_bytes)", scratch_bytes, need);
    if (!aligned16(scratch)) return fail("it_attn_f16: scratch must be 16-byte aligned");
    return check(it::launch_attn_splitk(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, ots, (float*)scratch, chunk, st),
                 "it_attn_f16 (split-K)");
}

int it_attn_f16_ex(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0, int hd, int nh,
                   int nkv, int nt, float scale, float* out, int ots, void* scratch, size_t scratch_bytes, int kernel,
                   int chunk, void* stream) {
    return attn_f16_impl(q, qts, nullptr, 0, kc, vc, kvd, pos0, hd, nh, nkv, nt, scale, out, ots, scratch,
                         scratch_bytes, kernel, chunk, stream);
}

int it_attn_f16_q16(const float* q, int qts, const uint16_t* q16, int q16ts, const uint16_t* kc, const uint16_t* vc,
                    int kvd, int pos0, int hd, int nh, int nkv, int nt, float scale, float* out, int ots, void* scratch,
                    size_t scratch_bytes, void* stream) {
    if (!q16) return fail("it_attn_f16_q16: null q16");
    if (!aligned16(q16) || q16ts % 8 != 0)
        return fail("it_attn_f16_q16: q16 must be 16-byte aligned, its token stride a multiple of 8");
    if (nt > 1 && q16ts < nh * hd) return fail("it_attn_f16_q16: q16 token stride %d overlaps rows", q16ts);
    return attn_f16_impl(q, qts, q16, q16ts, kc, vc, kvd, pos0, hd, nh, nkv, nt, scale, out, ots, scratch,
                         scratch_bytes, KERNEL_AUTO, 0, stream);
}

int it_attn_f16(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0, int hd, int nh,
                int nkv, int nt, float scale, float* out, int ots, void* scratch, size_t scratch_bytes, void* stream) {
    return it_attn_f16_ex(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, scale, out, ots, scratch, scratch_bytes,
                          KERNEL_AUTO, 0, stream);
}

int it_attn_f16_noalloc(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0, int hd,
                        int nh, int nkv, int nt, float scale, float* out, int ots, void* stream) {
    if (validate_attn(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, out, ots)) return -1;
    AttnPlan p;
    if (!plan_attn(pos0, nt, nh, nkv, KERNEL_AUTO, IT_NOALLOC_SCRATCH_BYTES, p))
        return fail("it_attn_f16_noalloc: this geometry needs %zu bytes of partial records, more than the %zu-byte "
                    "device scratch (use it_attn_f16 with a caller buffer)", p.bytes, (size_t)IT_NOALLOC_SCRATCH_BYTES);
    void* scr = nullptr;
    if (noalloc_scratch(&scr)) return -1;
    // the same launch path as it_attn_f16 with the plan fixed: no allocation anywhere below
    return it_attn_f16_ex(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, scale, out, ots, scr, IT_NOALLOC_SCRATCH_BYTES,
                          p.kernel, p.kernel == KERNEL_FLASH && p.chunk == 0 ? (1 << 30) : p.chunk, stream);
}

size_t it_attn_mailbox_bytes(int ctx, int nt, int nh) {
    if (ctx <= 0 || nt <= 0 || nh <= 0) return 0;
    return it::mailbox_bytes(ctx, nt, nh);
}

int it_attn_mailbox_init(void* mailbox, size_t bytes, void* stream) {
    if (!mailbox || bytes < it::mailbox_bytes(1, 1, 1) || bytes % 4) return fail("it_attn_mailbox_init: bad buffer");
    if (!aligned16(mailbox)) return fail("it_attn_mailbox_init: the mailbox must be 16-byte aligned");
    volatile uint32_t* host = nullptr;
    uint32_t* dev = nullptr;
    if (mailbox_report(mailbox, true, &host, &dev)) return -1;
    *host = 0;   // now, for the calls that follow; the fill clears it again in stream order
    return check(it::launch_mailbox_fill(mailbox, bytes, dev, (hipStream_t)stream), "it_attn_mailbox_init");
}

int it_attn_mailbox_poisoned(const void* mailbox, int* poisoned, void* stream) {
    if (!mailbox || !poisoned) return fail("it_attn_mailbox_poisoned: null argument");
    uint32_t w[2] = {0, 0};
    hipStream_t st = (hipStream_t)stream;
    if (check(hipMemcpyAsync(w, mailbox, 8, hipMemcpyDeviceToHost, st), "it_attn_mailbox_poisoned")) return -1;
    if (check(hipStreamSynchronize(st), "it_attn_mailbox_poisoned")) return -1;
    *poisoned = w[0] != 0 || w[1] != it::MAILBOX_MAGIC;   // gave up, or never initialised
    return 0;
}

int it_attn_mailbox_would_launch(int pos0, int nt, int hd, int nh, int nkv, size_t mailbox_bytes) {
    if (hd != HD || nt <= 0 || pos0 < 0 || nh <= 0 || nkv <= 0 || nh % nkv) return 0;
    if (auto_kernel(nt) != KERNEL_SPLITK) return 0;
    bool launched = false;
    float dummy;
    if (it::launch_attn_decode_mailbox(nullptr, 0, nullptr, nullptr, nkv * HD, pos0, nh, nkv, nt, 0.f, nullptr, 0,
                                       &dummy, mailbox_bytes, nullptr, &launched, true) != hipSuccess)
        return 0;
    return launched ? 1 : 0;
}

int it_attn_f16_mailbox(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0, int hd,
                        int nh, int nkv, int nt, float scale, float* out, int ots, void* mailbox, size_t mailbox_bytes,
                        void* scratch, size_t scratch_bytes, void* stream) {
    if (validate_attn(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, out, ots)) return -1;
    if (mailbox && !aligned16(mailbox)) return fail("it_attn_f16_mailbox: the mailbox must be 16-byte aligned");
    if (mailbox) {
        // an earlier call's merge found this mailbox poisoned (it gave up waiting, or the mailbox
        // was overwritten): fail before any device work instead of returning NaN again
        volatile uint32_t* host = nullptr;
        if (mailbox_report(mailbox, false, &host, nullptr)) return -1;
        if (host && *host)
            return fail("it_attn_f16_mailbox: the mailbox was found poisoned by an earlier call (a merge gave up "
                        "waiting); re-initialise it with it_attn_mailbox_init");
    }
    if (auto_kernel(nt) == KERNEL_SPLITK) {
        bool launched = false;
        if (check(it::launch_attn_decode_mailbox(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, out, ots,
                                                 (float*)mailbox, mailbox ? mailbox_bytes : 0, (hipStream_t)stream,
                                                 &launched),
                  "it_attn_f16_mailbox"))
            return -1;
        if (launched) return 0;
    }
    return it_attn_f16(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, scale, out, ots, scratch, scratch_bytes, stream);
}

int it_attn_partials(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0, int hd, int nh,
                     int nkv, int nt, float scale, float* part, size_t part_bytes, int chunk, void* stream) {
    if (validate_attn(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, q, qts)) return -1;
    if (chunk <= 0 || chunk % 64 != 0) return fail("it_attn_partials: chunk %d must be a positive multiple of 64", chunk);
    const size_t need = splitk_scratch(pos0, nt, nh, chunk);
    if (!part || part_bytes < need) return fail("it_attn_partials: %zu bytes of partials < %zu required", part_bytes, need);
    if (!aligned16(part)) return fail("it_attn_partials: part must be 16-byte aligned");
    return check(it::launch_attn_partials(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, (hipStream_t)stream),
                 "it_attn_partials");
}

int it_attn_combine(const float* q, int qts, const float* part, int pos0, int hd, int nh, int nt, int chunk, float* out,
                    int ots, void* stream) {
    if (hd != HD || nh <= 0 || nt <= 0 || pos0 < 0) return fail("it_attn_combine: bad geometry");
    if (chunk <= 0 || chunk % 64 != 0) return fail("it_attn_combine: chunk %d must be a positive multiple of 64", chunk);
    if (!q || !part || !out || !aligned16(q) || !aligned16(part) || !aligned16(out))
        return fail("it_attn_combine: buffers must be non-null and 16-byte aligned");
    if (qts % 4 != 0 || ots % 4 != 0) return fail("it_attn_combine: token strides must be multiples of 4");
    return check(it::launch_attn_combine(q, qts, part, pos0, nh, nt, chunk, out, ots, (hipStream_t)stream),
                 "it_attn_combine");
}

int it_attn_partials_ex(const float* q, int qts, const uint16_t* kc, const uint16_t* vc, int kvd, int pos0, int hd,
                        int nh, int nkv, int nt, float scale, float* part, size_t part_bytes, int chunk, int layout,
                        void* stream) {
    if (layout == 0) return it_attn_partials(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, scale, part, part_bytes, chunk, stream);
    if (layout != 1) return fail("it_attn_partials_ex: unknown record layout %d (0 or 1)", layout);
    if (validate_attn(q, qts, kc, vc, kvd, pos0, hd, nh, nkv, nt, q, qts)) return -1;
    if (chunk <= 0 || chunk % 64 != 0) return fail("it_attn_partials_ex: chunk %d must be a positive multiple of 64", chunk);
    if (!it::piece_records(pos0, nt, nh, chunk))
        return fail("it_attn_partials_ex: record layout 1 needs 9-256 splits and at most 256 (token, head) rows");
    const size_t need = splitk_scratch(pos0, nt, nh, chunk);
    if (!part || part_bytes < need) return fail("it_attn_partials_ex: %zu bytes of partials < %zu required", part_bytes, need);
    if (!aligned16(part)) return fail("it_attn_partials_ex: part must be 16-byte aligned");
    return check(it::launch_attn_partials(q, qts, kc, vc, kvd, pos0, nh, nkv, nt, scale, part, chunk, (hipStream_t)stream,
                                          true),
                 "it_attn_partials_ex");
}

int it_attn_combine_ex(const float* q, int qts, const float* part, int pos0, int hd, int nh, int nt, int chunk, int layout,
                       float* out, int ots, void* stream) {
    if (layout == 0) return it_attn_combine(q, qts, part, pos0, hd, nh, nt, chunk, out, ots, stream);
    if (layout != 1) return fail("it_attn_combine_ex: unknown record layout %d (0 or 1)", layout);
    if (hd != HD || nh <= 0 || nt <= 0 || pos0 < 0) return fail("it_attn_combine_ex: bad geometry");
    if (chunk <= 0 || chunk % 64 != 0) return fail("it_attn_combine_ex: chunk %d must be a positive multiple of 64", chunk);
    if (!it::piece_records(pos0, nt, nh, chunk))
        return fail("it_attn_combine_ex: record layout 1 needs 9-256 splits and at most 256 (token, head) rows");
    if (!q || !part || !out || !aligned16(q) || !aligned16(part) || !aligned16(out))
        return fail("it_attn_combine_ex: buffers must be non-null and 16-byte aligned");
    if (qts % 4 != 0 || ots % 4 != 0) return fail("it_attn_combine_ex: token strides must be multiples of 4");
    return check(it::launch_attn_combine(q, qts, part, pos0, nh, nt, chunk, out, ots, (hipStream_t)stream, true),
                 "it_attn_combine_ex");
}

int it_gdn_conv(const float* x, int xts, const float* w, float* state, float* out, int ots, int cd, int nt, int K,
                void* stream) {
    if (K < 2 || K > 4) return fail("it_gdn_conv: kernel size %d unsupported (2..4)", K);
    if (cd <= 0 || nt < 0) return fail("it_gdn_conv: bad geometry cd=%d nt=%d", cd, nt);
    if (nt > 1 && (xts < cd || ots < cd)) return fail("it_gdn_conv: token strides smaller than cd");
    if (!x || !w || !state || !out) return fail("it_gdn_conv: null buffer");
    if (nt == 0) { g_err.clear(); return 0; }
    return check(it::launch_gdn_conv(x, xts, w, state, out, ots, cd, nt, K, nullptr, 0, (hipStream_t)stream),
                 "it_gdn_conv");
}

// The checkpoint buffer must not overlap the live state (it is written while the state is read).
static int validate_ckpt(const char* who, const float* ck, const float* state, size_t words, int ck_after, int nt) {
    if (!ck) return fail("%s: null checkpoint buffer", who);
    if (ck_after < 0 || ck_after >= nt) return fail("%s: checkpoint token %d outside [0, %d)", who, ck_after, nt);
    if (ck < state + words && state < ck + words) return fail("%s: checkpoint buffer overlaps the state", who);
    return 0;
}

int it_gdn_conv_ckpt(const float* x, int xts, const float* w, float* state, float* out, int ots, int cd, int nt, int K,
                     float* ck_state, int ck_after, void* stream) {
    if (K < 2 || K > 4) return fail("it_gdn_conv_ckpt: kernel size %d unsupported (2..4)", K);
    if (cd <= 0 || nt <= 0) return fail("it_gdn_conv_ckpt: bad geometry cd=%d nt=%d", cd, nt);
    if (nt > 1 && (xts < cd || ots < cd)) return fail("it_gdn_conv_ckpt: token strides smaller than cd");
    if (!x || !w || !state || !out) return fail("it_gdn_conv_ckpt: null buffer");
    if (validate_ckpt("it_gdn_conv_ckpt", ck_state, state, (size_t)(K - 1) * cd, ck_after, nt)) return -1;
    return check(it::launch_gdn_conv(x, xts, w, state, out, ots, cd, nt, K, ck_state, ck_after, (hipStream_t)stream),
                 "it_gdn_conv_ckpt");
}

int it_gdn_conv_l2norm(const float* x, int xts, const float* w, float* state, float* out, int ots, int cd, int nt, int K,
                       int nnorm, float eps, void* stream) {
    if (K < 2 || K > 4) return fail("it_gdn_conv_l2norm: kernel size %d unsupported (2..4)", K);
    if (cd <= 0 || cd % 128 != 0 || nt < 0) return fail("it_gdn_conv_l2norm: bad geometry cd=%d nt=%d (cd a multiple of 128)", cd, nt);
    if (nnorm < 0 || nnorm * 128 > cd) return fail("it_gdn_conv_l2norm: %d normalised heads exceed cd=%d", nnorm, cd);
    if (nt > 1 && (xts < cd || ots < cd)) return fail("it_gdn_conv_l2norm: token strides smaller than cd");
    if (!x || !w || !state || !out) return fail("it_gdn_conv_l2norm: null buffer");
    if (nt == 0) { g_err.clear(); return 0; }
    return check(it::launch_gdn_conv_l2(x, xts, w, state, out, ots, cd, nt, K, nnorm, eps, nullptr, 0,
                                        (hipStream_t)stream),
                 "it_gdn_conv_l2norm");
}

int it_gdn_conv_l2norm_ckpt(const float* x, int xts, const float* w, float* state, float* out, int ots, int cd, int nt,
                            int K, int nnorm, float eps, float* ck_state, int ck_after, void* stream) {
    const char* who = "it_gdn_conv_l2norm_ckpt";
    if (K < 2 || K > 4) return fail("%s: kernel size %d unsupported (2..4)", who, K);
    if (cd <= 0 || cd % 128 != 0 || nt <= 0) return fail("%s: bad geometry cd=%d nt=%d (cd a multiple of 128)", who, cd, nt);
    if (nnorm < 0 || nnorm * 128 > cd) return fail("%s: %d normalised heads exceed cd=%d", who, nnorm, cd);
    if (nt > 1 && (xts < cd || ots < cd)) return fail("%s: token strides smaller than cd", who);
    if (!x || !w || !state || !out) return fail("%s: null buffer", who);
    if (validate_ckpt(who, ck_state, state, (size_t)(K - 1) * cd, ck_after, nt)) return -1;
    return check(it::launch_gdn_conv_l2(x, xts, w, state, out, ots, cd, nt, K, nnorm, eps, ck_state, ck_after,
                                        (hipStream_t)stream),
                 who);
}

int it_l2norm_heads(float* x, int ts, int nheads, int d, int nt, float eps, void* stream) {
    if (d != 128 && d != 256) return fail("it_l2norm_heads: row length %d unsupported (128 or 256)", d);
    if (nheads <= 0 || nt < 0) return fail("it_l2norm_heads: bad geometry");
    if (nt > 1 && ts < nheads * d) return fail("it_l2norm_heads: token stride overlaps rows");
    if (!x) return fail("it_l2norm_heads: null buffer");
    if (nt == 0) { g_err.clear(); return 0; }
    return check(it::launch_l2norm(x, ts, nheads, d, nt, eps, (hipStream_t)stream), "it_l2norm_heads");
}

static int validate_gdn(const char* who, const float* co, int cts, const float* br, const float* ar, int bts,
                        const float* dt, const float* a, const float* state, const float* out, int ots, int nt, int nv,
                        int nk, int S) {
    if (S != 128) return fail("%s: state size %d unsupported (128)", who, S);
    if (nv <= 0 || nk <= 0 || nv % nk != 0) return fail("%s: nv %d / nk %d invalid", who, nv, nk);
    if (nt < 0) return fail("%s: nt %d invalid", who, nt);
    if (!co || !br || !ar || !dt || !a || !state || !out) return fail("%s: null buffer", who);
    if (!aligned16(co) || !aligned16(state) || !aligned16(out)) return fail("%s: co/state/out must be 16-byte aligned", who);
    if (cts % 4 != 0 || ots % 4 != 0) return fail("%s: token strides must be multiples of 4", who);
    if (nt > 1 && (cts < (2 * nk + nv) * S || ots < nv * S || bts < nv)) return fail("%s: token strides overlap rows", who);
    return 0;
}

int it_gdn_step(const float* co, int cts, const float* br, const float* ar, int bts, const float* dt, const float* a,
                float* state, float* out, int ots, int nt, int nv, int nk, int S, void* stream) {
    if (validate_gdn("it_gdn_step", co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, S)) return -1;
    if (nt == 0) { g_err.clear(); return 0; }
    return check(it::launch_gdn_step(co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, nullptr, 0,
                                     (hipStream_t)stream),
                 "it_gdn_step");
}

static int validate_decode_fused(const char* who, const float* x, int xts, const float* w, int K, const float* cst_in,
                                 const float* cst_out, const float* br, const float* ar, int bts, const float* dt,
                                 const float* a, const float* state, const float* out, int ots, int nt, int nv, int nk,
                                 int S) {
    if (S != 128) return fail("%s: state size %d unsupported (128)", who, S);
    if (nv <= 0 || nk <= 0 || nv % nk != 0) return fail("%s: nv %d / nk %d invalid", who, nv, nk);
    if (nt < 1 || nt > 4) return fail("%s: nt %d outside 1..4 (longer runs: it_gdn_conv_l2norm + it_gdn_step)", who, nt);
    if (K < 2 || K > 4) return fail("%s: kernel size %d unsupported (2..4)", who, K);
    if (!x || !w || !cst_in || !cst_out || !br || !ar || !dt || !a || !state || !out) return fail("%s: null buffer", who);
    const int cd = (2 * nk + nv) * S;
    if (!aligned16(x) || !aligned16(w) || !aligned16(cst_in) || !aligned16(cst_out) || !aligned16(state) ||
        !aligned16(out))
        return fail("%s: x / w / conv states / state / out must be 16-byte aligned", who);
    if (xts % 4 != 0 || ots % 4 != 0) return fail("%s: token strides must be multiples of 4", who);
    if (nt > 1 && (xts < cd || ots < nv * S || bts < nv)) return fail("%s: token strides overlap rows", who);
    const size_t cbytes = (size_t)(K - 1) * cd * sizeof(float);
    const char *pi = (const char*)cst_in, *po = (const char*)cst_out;
    if (pi < po + cbytes && po < pi + cbytes) return fail("%s: conv_state_out overlaps conv_state_in", who);
    return 0;
}

int it_gdn_decode_fused(const float* x, int xts, const float* w, int K, const float* cst_in, float* cst_out,
                        const float* br, const float* ar, int bts, const float* dt, const float* a, float* state,
                        float* out, int ots, int nt, int nv, int nk, int S, float eps, void* stream) {
    const char* who = "it_gdn_decode_fused";
    if (validate_decode_fused(who, x, xts, w, K, cst_in, cst_out, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, S))
        return -1;
    return check(it::launch_gdn_decode_fused(x, xts, w, K, cst_in, cst_out, br, ar, bts, dt, a, state, out, ots, nt, nv,
                                             nk, eps, nullptr, nullptr, -1, (hipStream_t)stream),
                 who);
}

int it_gdn_decode_fused_ckpt(const float* x, int xts, const float* w, int K, const float* cst_in, float* cst_out,
                             const float* br, const float* ar, int bts, const float* dt, const float* a, float* state,
                             float* out, int ots, int nt, int nv, int nk, int S, float eps, float* ck_state,
                             float* ck_conv, int ck_after, void* stream) {
    const char* who = "it_gdn_decode_fused_ckpt";
    if (validate_decode_fused(who, x, xts, w, K, cst_in, cst_out, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, S))
        return -1;
    if (validate_ckpt(who, ck_state, state, (size_t)nv * S * S, ck_after, nt)) return -1;
    const size_t cwords = (size_t)(K - 1) * (2 * nk + nv) * S;
    if (validate_ckpt(who, ck_conv, cst_in, cwords, ck_after, nt)) return -1;
    if (ck_conv < cst_out + cwords && cst_out < ck_conv + cwords) return fail("%s: conv checkpoint overlaps the conv state", who);
    if (!aligned16(ck_state) || !aligned16(ck_conv)) return fail("%s: checkpoint buffers must be 16-byte aligned", who);
    return check(it::launch_gdn_decode_fused(x, xts, w, K, cst_in, cst_out, br, ar, bts, dt, a, state, out, ots, nt, nv,
                                             nk, eps, ck_state, ck_conv, ck_after, (hipStream_t)stream),
                 who);
}

int it_gdn_step_ckpt(const float* co, int cts, const float* br, const float* ar, int bts, const float* dt,
                     const float* a, float* state, float* out, int ots, int nt, int nv, int nk, int S, float* ck_state,
                     int ck_after, void* stream) {
    if (validate_gdn("it_gdn_step_ckpt", co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, S)) return -1;
    if (validate_ckpt("it_gdn_step_ckpt", ck_state, state, (size_t)nv * S * S, ck_after, nt)) return -1;
    if (!aligned16(ck_state)) return fail("it_gdn_step_ckpt: checkpoint buffer must be 16-byte aligned");
    return check(it::launch_gdn_step(co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, ck_state, ck_after,
                                     (hipStream_t)stream),
                 "it_gdn_step_ckpt");
}

int it_gdn_step_gated(const float* co, int cts, const float* br, const float* ar, int bts, const float* dt,
                      const float* a, float* state, float* out, int ots, int nt, int nv, int nk, int S, const float* z,
                      int zts, const float* norm_w, float eps, float* ck_state, int ck_after, void* stream) {
    const char* who = "it_gdn_step_gated";
    if (validate_gdn(who, co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, S)) return -1;
    if (z) {
        if (!norm_w) return fail("%s: null norm weight", who);
        if (!aligned16(z) || !aligned16(norm_w) || zts % 4 != 0) return fail("%s: z / norm_w must be 16-byte aligned", who);
        if (nt > 1 && zts < nv * S) return fail("%s: z token stride overlaps rows", who);
        if (!(eps >= 0.0f)) return fail("%s: eps must be >= 0", who);
    }
    if (ck_state) {
        if (validate_ckpt(who, ck_state, state, (size_t)nv * S * S, ck_after, nt)) return -1;
        if (!aligned16(ck_state)) return fail("%s: checkpoint buffer must be 16-byte aligned", who);
    }
    if (nt == 0) { g_err.clear(); return 0; }
    return check(it::launch_gdn_step_head(co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, z, zts, norm_w, eps,
                                          ck_state, ck_state ? ck_after : 0, (hipStream_t)stream),
                 who);
}

int it_gdn_gated_rmsnorm(const float* o, int ots, const float* z, int zts, const float* w, float eps, float* out,
                         int outs, int nv, int S, int nt, void* stream) {
    const char* who = "it_gdn_gated_rmsnorm";
    if (S != 128) return fail("%s: head size %d unsupported (128)", who, S);
    if (nv <= 0 || nt < 0) return fail("%s: bad geometry nv=%d nt=%d", who, nv, nt);
    if (!o || !z || !w || !out) return fail("%s: null buffer", who);
    if (nt > 1 && (ots < nv * S || zts < nv * S || outs < nv * S)) return fail("%s: token strides overlap rows", who);
    if (out != o && out < o + (size_t)(nt ? nt - 1 : 0) * ots + (size_t)nv * S && o < out + (size_t)(nt ? nt - 1 : 0) * outs + (size_t)nv * S)
        return fail("%s: out must be o itself or not overlap it", who);
    if (!(eps >= 0.0f)) return fail("%s: eps must be >= 0", who);
    if (nt == 0) { g_err.clear(); return 0; }
    return check(it::launch_gdn_gated_norm(o, ots, z, zts, w, eps, out, outs, nv, nt, (hipStream_t)stream), who);
}

int it_gdn_rollback(const float* ck_conv, float* conv_state, size_t conv_words, const float* ck_ssm, float* ssm,
                    size_t ssm_words, void* stream) {
    if ((conv_words && (!ck_conv || !conv_state)) || (ssm_words && (!ck_ssm || !ssm)))
        return fail("it_gdn_rollback: null buffer");
    if (!conv_words && !ssm_words) { g_err.clear(); return 0; }
    return check(it::launch_gdn_rollback(ck_conv, conv_state, conv_words, ck_ssm, ssm, ssm_words, (hipStream_t)stream),
                 "it_gdn_rollback");
}

size_t it_gdn_chunked_scratch_bytes(int nt, int nv, int S) {
    if (nt <= 0 || nv <= 0 || S != 128) return 0;
    return it::gdn_chunked_scratch_bytes(nt, nv, S, false);
}

int it_gdn_chunked(const float* co, int cts, const float* br, const float* ar, int bts, const float* dt, const float* a,
                   float* state, float* out, int ots, int nt, int nv, int nk, int S, void* scratch, size_t scratch_bytes,
                   void* stream) {
    if (validate_gdn("it_gdn_chunked", co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, S)) return -1;
    if (nt == 0) { g_err.clear(); return 0; }
    const size_t need = it::gdn_chunked_scratch_bytes(nt, nv, S, false);
    if (scratch_bytes < need || (need && !scratch))
        return fail("it_gdn_chunked: scratch of %zu bytes < %zu required", scratch_bytes, need);
    if (!aligned16(scratch)) return fail("it_gdn_chunked: scratch must be 16-byte aligned");
    return check(it::launch_gdn_chunked(co, cts, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, scratch,
                                        (hipStream_t)stream),
                 "it_gdn_chunked");
}

static size_t gdn_prefill_co_bytes(int nt, int nv, int nk, int S) {
    return ((size_t)nt * (size_t)(2 * nk + nv) * S * 2 + 255) / 256 * 256;
}

size_t it_gdn_prefill_scratch_bytes(int nt, int nv, int nk, int S) {
    if (nt <= 0 || nv <= 0 || nk <= 0 || S != 128) return 0;
    return gdn_prefill_co_bytes(nt, nv, nk, S) + it::gdn_chunked_scratch_bytes(nt, nv, S, true);
}

int it_gdn_prefill(const float* x, int xts, const float* w, int K, float* conv_state, const float* br, const float* ar,
                   int bts, const float* dt, const float* a, float* state, float* out, int ots, int nt, int nv,
                   int nk, int S, float eps, void* scratch, size_t scratch_bytes, void* stream) {
    const char* who = "it_gdn_prefill";
    if (K < 2 || K > 4) return fail("%s: kernel size %d unsupported (2..4)", who, K);
    if (S != 128) return fail("%s: state size %d unsupported (128)", who, S);
    if (nv <= 0 || nk <= 0 || nv % nk != 0) return fail("%s: nv %d / nk %d invalid", who, nv, nk);
    if (nt < 0) return fail("%s: nt %d invalid", who, nt);
    if (!x || !w || !conv_state || !br || !ar || !dt || !a || !state || !out) return fail("%s: null buffer", who);
    const int cd = (2 * nk + nv) * S;
    if (nt > 1 && (xts < cd || ots < nv * S || bts < nv)) return fail("%s: token strides overlap rows", who);
    if (!aligned16(state) || !aligned16(out) || ots % 4 != 0)
        return fail("%s: state/out must be 16-byte aligned, the out token stride a multiple of 4", who);
    if (nt == 0) { g_err.clear(); return 0; }
    const size_t need = it_gdn_prefill_scratch_bytes(nt, nv, nk, S);
    if (scratch_bytes < need || !scratch)
        return fail("%s: scratch of %zu bytes < %zu required (it_gdn_prefill_scratch_bytes)", who, scratch_bytes, need);
    if (!aligned16(scratch)) return fail("%s: scratch must be 16-byte aligned", who);
    // the conv + SiLU + q/k L2 output goes to the front of the scratch as f16 (token stride cd),
    // the chunk records after it
    _Float16* co = (_Float16*)scratch;
    void* rec = (char*)scratch + gdn_prefill_co_bytes(nt, nv, nk, S);
    hipStream_t st = (hipStream_t)stream;
    if (check(it::launch_gdn_conv_l2(x, xts, w, conv_state, co, cd, cd, nt, K, 2 * nk, eps, nullptr, 0, st), who))
        return -1;
    return check(it::launch_gdn_chunked(co, cd, br, ar, bts, dt, a, state, out, ots, nt, nv, nk, rec, st), who);
}

// ---- reference-shaped policy (src/vk/mod.rs:130-220) -------------------------------------------
size_t it_attention_scratch_words(size_t ctx, size_t heads) { return 64 * heads * (ctx > 260 ? ctx : 260); }

size_t it_attention_dispatch_room(size_t ctx, size_t heads, size_t nt) {
    if (nt == 0 || nt > 512) return 0;
    return (nt + 63) / 64 * 64 * heads * (ctx > 260 ? ctx : 260);
}

int it_attention_chunk(uint32_t nt, uint32_t nh, uint32_t pos0, size_t room) {
    const uint64_t total = (uint64_t)pos0 + nt;
    uint64_t c = 64;
    while (c < 1024 && (uint64_t)nt * nh * ((total + c - 1) / c) * 260 > room) c *= 2;
    if ((uint64_t)nt * nh * ((total + c - 1) / c) * 260 > room) return -1;
    return (int)c;
}

long it_prefill_chunks(size_t len, size_t batch, size_t* starts, size_t* lens, size_t cap) {
    if (batch != 64 && batch != 128 && batch != 256 && batch != 512)
        return fail("it_prefill_chunks: unsupported prefill batch %zu; use 64/128/256/512", batch), -1;
    long count = 0;
    for (size_t start = 0; start < len;) {
        size_t n = len - start < batch ? len - start : batch;
        const size_t tail = n % 64;
        if (n > 64 && tail > 0 && tail < 22) n -= tail;   // the short tail goes to the next range
        if ((size_t)count < cap) {
            if (starts) starts[count] = start;
            if (lens) lens[count] = n;
        }
        ++count;
        start += n;
    }
    g_err.clear();
    return count;
}

int it_validate_geometry(int ctx_len, int head_dim, int n_head, int n_head_kv, int ssm_state, int ssm_groups,
                         int ssm_vheads, int ssm_inner, int conv_k) {
    if (ctx_len <= 0 || ctx_len > 8192) return fail("supported context capacity is 1..=8192");
    if (head_dim != 256 || n_head <= 0 || n_head_kv <= 0 || n_head % n_head_kv != 0 || ssm_state != 128 ||
        ssm_groups <= 0 || ssm_vheads <= 0 || ssm_vheads % ssm_groups != 0 || ssm_inner != ssm_vheads * ssm_state ||
        ssm_inner % 1024 != 0 || conv_k < 2 || conv_k > 4)
        return fail("unsupported kernel geometry");
    g_err.clear();
    return 0;
}

int it_calib_mfma_f16(int wgs, int iters, float* out, void* stream) {
    if (wgs < 1 || iters < 1 || !out) return fail("it_calib_mfma_f16: wgs %d / iters %d / out invalid", wgs, iters);
    return check(it::launch_mfma_peak(wgs, iters, out, (hipStream_t)stream), "it_calib_mfma_f16");
}

}  // extern "C"
