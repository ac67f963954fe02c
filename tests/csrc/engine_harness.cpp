// Engine-shaped C++ caller of the C ABI (include/it_attn.h), the way the reference's Vulkan engine
// drives its attention and Gated-DeltaNet dispatches (src/vk/mod.rs:544-566, 790-806, 839, 896):
// one caller-owned device arena addressed by word offsets, a prompt split by prefill_chunks
// (it_prefill_chunks, vk/mod.rs:130-134), each attention call given exactly the arena room the
// reference reserves for its dispatch (attention_dispatch_room, vk/mod.rs:148) as scratch, then
// decode tokens one at a time: attention through it_attn_f16 with the same room, the one-launch
// GDN layer with its ping-pong conv state. The MTP head's attention over an f32 cache (vk/mod.rs:942)
// runs over the same tokens in 64-token catch-up calls (effective_prefill_batch, vk/mod.rs:143-146),
// each given the dispatch room as scratch too.
//
// Test driver only (tests/test_gpu_engine_harness.py builds the inputs and checks the outputs
// against the oracle). Usage: engine_harness DIR T_PROMPT T_DECODE UBATCH
//   DIR holds q.bin k.bin v.bin (attention inputs, f32 [T][...]) and x.bin w.bin cst.bin st.bin
//   br.bin ar.bin dt.bin a.bin (GDN inputs); attn_out.bin gdn_out.bin state_out.bin cst_out.bin
//   mtp_out.bin are written back. Geometry: 16 q / 2 KV heads, head_dim 256; 32 V / 16 QK heads, state 128, conv 4.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../include/it_attn.h"

namespace {

constexpr int NH = 16, NKV = 2, HD = 256, KVD = NKV * HD, QTS = NH * 2 * HD, OTS = NH * HD;
constexpr int NV = 32, NK = 16, S = 128, CD = (2 * NK + NV) * S, KC = 4;
constexpr float EPS = 1e-6f;

#define HIPCHECK(x)                                                                                  \
    do {                                                                                             \
        hipError_t e_ = (x);                                                                         \
        if (e_ != hipSuccess) {                                                                      \
            std::fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            std::exit(2);                                                                            \
        }                                                                                            \
    } while (0)
#define ITCHECK(x)                                                                              \
    do {                                                                                        \
        if ((x) != 0) {                                                                         \
            std::fprintf(stderr, "%s:%d %s failed: %s\n", __FILE__, __LINE__, #x, it_last_error()); \
            std::exit(3);                                                                       \
        }                                                                                       \
    } while (0)

std::vector<float> read_file(const std::string& path, size_t n) {
    std::vector<float> v(n);
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f || std::fread(v.data(), sizeof(float), n, f) != n) {
        std::fprintf(stderr, "cannot read %zu floats from %s\n", n, path.c_str());
        std::exit(4);
    }
    std::fclose(f);
    return v;
}
void write_file(const std::string& path, const float* d, size_t n) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(d, sizeof(float), n, f) != n) {
        std::fprintf(stderr, "cannot write %s\n", path.c_str());
        std::exit(4);
    }
    std::fclose(f);
}

// Word offsets into the arena (f32 words; the f16 KV caches take kvd/2 words a position).
struct Layout {
    size_t q, k, v, kc, vc, aout, scr, mout, x, w, cst0, cst1, st, br, ar, dt, a, gout, gscr, words;
};

}  // namespace

int main(int argc, char** argv) {
    if (argc < 5) {
        std::fprintf(stderr, "usage: engine_harness DIR T_PROMPT T_DECODE UBATCH\n");
        return 1;
    }
    const std::string dir = argv[1];
    const int tp = std::atoi(argv[2]), td = std::atoi(argv[3]), ub = std::atoi(argv[4]);
    const int T = tp + td, ctx = T;   // context capacity of the engine = the whole sequence

    Layout L{};
    size_t o = 0;
    auto take = [&](size_t words) { const size_t at = o; o += (words + 63) / 64 * 64; return at; };
    L.q = take((size_t)T * QTS);
    L.k = take((size_t)T * KVD);
    L.v = take((size_t)T * KVD);
    L.kc = take((size_t)ctx * KVD / 2);
    L.vc = take((size_t)ctx * KVD / 2);
    L.aout = take((size_t)T * OTS);
    // the arena's attention scratch: ubatch x heads x max(ctx, 260) words (vk/mod.rs:546), which is
    // the dispatch room of the largest chunk; it_attention_scratch_words is only the 64-token case
    L.scr = take(it_attention_dispatch_room(ctx, NH, ub));
    L.mout = take((size_t)T * OTS);   // the MTP head's attention output
    L.x = take((size_t)T * CD);
    L.w = take((size_t)CD * KC);
    L.cst0 = take((size_t)(KC - 1) * CD);
    L.cst1 = take((size_t)(KC - 1) * CD);
    L.st = take((size_t)NV * S * S);
    L.br = take((size_t)T * NV);
    L.ar = take((size_t)T * NV);
    L.dt = take(NV);
    L.a = take(NV);
    L.gout = take((size_t)T * NV * S);
    L.gscr = take((it_gdn_prefill_scratch_bytes(ub, NV, NK, S) + 3) / 4);   // f16 conv output + chunk records
    L.words = o;

    float* arena = nullptr;
    HIPCHECK(hipMalloc(&arena, L.words * sizeof(float)));
    hipStream_t s;
    HIPCHECK(hipStreamCreate(&s));
    auto up = [&](size_t off, const char* name, size_t n) {
        const std::vector<float> h = read_file(dir + "/" + name, n);
        HIPCHECK(hipMemcpy(arena + off, h.data(), n * sizeof(float), hipMemcpyHostToDevice));
    };
    up(L.q, "q.bin", (size_t)T * QTS);
    up(L.k, "k.bin", (size_t)T * KVD);
    up(L.v, "v.bin", (size_t)T * KVD);
    up(L.x, "x.bin", (size_t)T * CD);
    up(L.w, "w.bin", (size_t)CD * KC);
    up(L.cst0, "cst.bin", (size_t)(KC - 1) * CD);
    up(L.st, "st.bin", (size_t)NV * S * S);
    up(L.br, "br.bin", (size_t)T * NV);
    up(L.ar, "ar.bin", (size_t)T * NV);
    up(L.dt, "dt.bin", NV);
    up(L.a, "a.bin", NV);

    auto a = [&](size_t off) { return arena + off; };
    uint16_t* kc = (uint16_t*)(arena + L.kc);
    uint16_t* vc = (uint16_t*)(arena + L.vc);
    const size_t gscr_bytes = it_gdn_prefill_scratch_bytes(ub, NV, NK, S);

    // one attention layer call for tokens [t0, t0 + nt) with the dispatch room as scratch
    auto attention = [&](int t0, int nt) {
        const size_t room = it_attention_dispatch_room(ctx, NH, nt) * sizeof(float);
        ITCHECK(it_kv_append_f16(a(L.k + (size_t)t0 * KVD), a(L.v + (size_t)t0 * KVD), KVD, kc, vc, t0, nt, KVD, 0, s));
        ITCHECK(it_attn_f16(a(L.q + (size_t)t0 * QTS), QTS, kc, vc, KVD, t0, HD, NH, NKV, nt, 0.0625f,
                            a(L.aout + (size_t)t0 * OTS), OTS, a(L.scr), room, s));
    };

    // ---- prefill: the reference's chunk loop (vk/mod.rs:896)
    const long nr = it_prefill_chunks(tp, ub, nullptr, nullptr, 0);
    if (nr < 0) { std::fprintf(stderr, "it_prefill_chunks: %s\n", it_last_error()); return 3; }
    std::vector<size_t> starts(nr > 0 ? nr : 1), lens(nr > 0 ? nr : 1);
    it_prefill_chunks(tp, ub, starts.data(), lens.data(), nr);
    for (long i = 0; i < nr; ++i) {
        const int t0 = (int)starts[i], nt = (int)lens[i];
        attention(t0, nt);
        // GDN layer: conv + q/k L2 (vk/mod.rs:803-804) and the recurrence (806) in one call, the conv
        // output kept as f16 in the layer's scratch slot
        ITCHECK(it_gdn_prefill(a(L.x + (size_t)t0 * CD), CD, a(L.w), KC, a(L.cst0), a(L.br + (size_t)t0 * NV),
                               a(L.ar + (size_t)t0 * NV), NV, a(L.dt), a(L.a), a(L.st), a(L.gout + (size_t)t0 * NV * S),
                               NV * S, nt, NV, NK, S, EPS, a(L.gscr), gscr_bytes, s));
    }
    // ---- decode: one token per call; the GDN layer in one launch with the conv state alternating
    // between two arena slots
    int p = 0;
    for (int t = tp; t < T; ++t) {
        attention(t, 1);
        ITCHECK(it_gdn_decode_fused(a(L.x + (size_t)t * CD), CD, a(L.w), KC, a(p ? L.cst1 : L.cst0), a(p ? L.cst0 : L.cst1),
                                    a(L.br + (size_t)t * NV), a(L.ar + (size_t)t * NV), NV, a(L.dt), a(L.a), a(L.st),
                                    a(L.gout + (size_t)t * NV * S), NV * S, 1, NV, NK, S, EPS, s));
        p ^= 1;
    }
    // ---- MTP head catch-up: its attention over an f32 cache (here the f32 k/v rows themselves) in
    // calls of at most 64 tokens, each with the dispatch room of the arena as scratch
    for (int t0 = 0; t0 < T; t0 += 64) {
        const int nt = T - t0 < 64 ? T - t0 : 64;
        const size_t room = it_attention_dispatch_room(ctx, NH, nt) * sizeof(float);
        ITCHECK(it_attn_f32kv(a(L.q + (size_t)t0 * QTS), QTS, a(L.k), a(L.v), KVD, t0, HD, NH, NKV, nt, 0.0625f,
                              a(L.mout + (size_t)t0 * OTS), OTS, a(L.scr), room, s));
    }
    HIPCHECK(hipStreamSynchronize(s));

    auto down = [&](size_t off, const char* name, size_t n) {
        std::vector<float> h(n);
        HIPCHECK(hipMemcpy(h.data(), arena + off, n * sizeof(float), hipMemcpyDeviceToHost));
        write_file(dir + "/" + name, h.data(), n);
    };
    down(L.aout, "attn_out.bin", (size_t)T * OTS);
    down(L.gout, "gdn_out.bin", (size_t)T * NV * S);
    down(L.st, "state_out.bin", (size_t)NV * S * S);
    down(p ? L.cst1 : L.cst0, "cst_out.bin", (size_t)(KC - 1) * CD);
    down(L.mout, "mtp_out.bin", (size_t)T * OTS);
    std::printf("ok %ld prefill calls, %d decode steps, arena %zu MiB\n", nr, td, L.words * 4 >> 20);
    HIPCHECK(hipFree(arena));
    return 0;
}
