// TEST INFRASTRUCTURE ONLY -- the CPU oracle for the attention / Gated-DeltaNet hot path.
//
// Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
// only as the checker or the timed CPU baseline. The product path (libit_attn.so) never links it.
//
// This is a restatement, read as text, of the reference's CPU forward pass (src/cpu.rs), which is
// Rust and cannot be compiled in this image (no cargo/rustc). Each function cites the lines it
// follows. Arithmetic order within a head is kept: sequential f32 sums (Rust's Iterator::sum is a
// left fold from 0.0), no FMA contraction (built with -ffp-contract=off), expf/logf from libm in
// place of f32::exp/ln. Heads run on std::thread in place of rayon (cpu.rs:218, 264); rayon does not
// change the per-head summation order.
//
// Parity pins for every function are listed in the test files (tests/test_oracle_*.py):
//   it_ref_attn, it_ref_attn_f32kv -- r012 f64 known-answer sweep (src/vk/r012_parity.rs:6-28), closed forms
//                        (single key, equal scores), torch SDPA, split/chunk invariance.
//   it_ref_gdn_*      -- brute-force float64 recurrence, closed forms (beta=0, g -> -inf),
//                        conv over T tokens == T single-token calls.
//   it_ref_rope, it_ref_attn_prep -- pos 0 = identity, a single pair = the 2-D rotation by pos,
//                        the sector rule's fixed dims, pair norms, relative-position invariance of
//                        q.k, and an f64 statement with exact angles (error bounded by the f32
//                        angle recurrence); it_ref_rmsnorm -- unit RMS, constant rows.
//   it_ref_gdn_gated_norm -- z = 0 gives 0, large z gives rmsnorm(o)*w*z, constant rows, an f64
//                        statement.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>
#include <algorithm>

namespace {

// cpu.rs:19-21
inline float silu(float x) { return x / (1.0f + std::exp(-x)); }
inline float sigmoid(float x) { return 1.0f / (1.0f + std::exp(-x)); }
inline float softplus(float x) { return x > 20.0f ? x : std::log(1.0f + std::exp(x)); }

// Half -> float (exact).
inline float h2f(uint16_t h) {
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023, bits;
    if (e == 0) {
        if (m == 0) bits = s;
        else { // subnormal: renormalise
            int sh = 0; while (!(m & 1024)) { m <<= 1; ++sh; }
            bits = s | ((uint32_t)(113 - sh) << 23) | ((m & 1023) << 13);
        }
    } else if (e == 31) bits = s | 0x7f800000u | (m << 13);
    else bits = s | ((e + 112) << 23) | (m << 13);
    float f; std::memcpy(&f, &bits, 4); return f;
}

template <class F> void par_for(int n, int threads, F f) {
    if (threads <= 1 || n <= 1) { for (int i = 0; i < n; ++i) f(i); return; }
    std::vector<std::thread> ts; int nt = std::min(threads, n);
    for (int w = 0; w < nt; ++w) ts.emplace_back([=, &f] { for (int i = w; i < n; i += nt) f(i); });
    for (auto& t : ts) t.join();
}

} // namespace

extern "C" {

int it_ref_hardware_threads() { return (int)std::max(1u, std::thread::hardware_concurrency()); }

// The kernel-parity harness's input generator (src/vk/kparity.rs:13, Rng::f): xorshift64 with shifts
// 13, 7, 17, then the top 24 bits of the state scaled to [-1, 1). Fills out[0..n) starting from
// *state and leaves the advanced state in *state, so the arena draw (kparity.rs:61) followed by
// the params draw (kparity.rs:62) is two calls.
void it_ref_xorshift_fill(uint64_t* state, size_t n, float* out) {
    uint64_t x = *state;
    for (size_t i = 0; i < n; ++i) {
        x ^= x << 13;
        x ^= x >> 7;
        x ^= x << 17;
        out[i] = ((float)(x >> 40) / (float)(1u << 24)) * 2.0f - 1.0f;
    }
    *state = x;
}

// f32 -> f16 bits, round to nearest even (the `half` crate's f16::from_f32, cpu.rs:22).
uint16_t it_ref_f32_to_f16_rne(float x) {
    uint32_t b; std::memcpy(&b, &x, 4);
    uint32_t s = (b >> 16) & 0x8000u; int32_t e = (int32_t)((b >> 23) & 0xff); uint32_t m = b & 0x7fffffu;
    if (e == 0xff) return (uint16_t)(s | 0x7c00u | (m ? 0x200u | (m >> 13) : 0));
    int32_t he = e - 127 + 15;
    if (he >= 31) return (uint16_t)(s | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return (uint16_t)s;
        m |= 0x800000u; uint32_t shift = (uint32_t)(14 - he);
        uint32_t hm = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1))) ++hm;
        return (uint16_t)(s | hm);
    }
    uint32_t hm = m >> 13, rem = m & 0x1fffu;
    uint32_t out = s | ((uint32_t)he << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1))) ++out; // carry may roll into exponent: correct
    return (uint16_t)out;
}
float it_ref_f16_to_f32(uint16_t h) { return h2f(h); }

// cpu.rs:14-18 rmsnorm with weight w (pass w = nullptr for unit weight).
void it_ref_rmsnorm(const float* x, const float* w, int n, float eps, float* y) {
    float ss = 0.0f; for (int i = 0; i < n; ++i) ss += x[i] * x[i];
    ss = ss / (float)n;
    float s = 1.0f / std::sqrt(ss + eps);
    for (int i = 0; i < n; ++i) y[i] = x[i] * s * (w ? w[i] : 1.0f);
}

// cpu.rs:147 theta_scale = base^(-2 / n_rot), f32 (the value the reference pushes, vk/mod.rs:824).
float it_ref_rope_theta_scale(float base, int n_rot) { return std::pow(base, -2.0f / (float)n_rot); }

// cpu.rs:145-162 neox-style (I)MRoPE in place on nheads rows of head_dim floats at position pos:
// the angle of frequency i is the f32 recurrence theta_0 = pos, theta_{i+1} = theta_i * theta_scale,
// replaced by 0 for a frequency whose sector lies outside the text sections.
void it_ref_rope(float* x, int nheads, int head_dim, int n_rot, int pos, float base, const int* sections) {
    const int half = n_rot / 2;
    const float theta_scale = it_ref_rope_theta_scale(base, n_rot);
    const int sect = sections[0] + sections[1] + sections[2] + sections[3];
    for (int h = 0; h < nheads; ++h) {
        float* r = x + (size_t)h * head_dim;
        float theta = (float)pos;
        for (int i = 0; i < half; ++i) {
            const int sector = sect > 0 ? i % sect : 0;
            const bool use_e = sect > 0 && !((sector % 3 == 1 && sector < 3 * sections[1]) ||
                                             (sector % 3 == 2 && sector < 3 * sections[2]) ||
                                             (sector % 3 == 0 && sector < 3 * sections[0]));
            const float th = use_e ? 0.0f : theta;
            const float sn = std::sin(th), c = std::cos(th);
            const float x0 = r[i], x1 = r[i + half];
            r[i] = x0 * c - x1 * sn;
            r[i + half] = x0 * sn + x1 * c;
            theta *= theta_scale;
        }
    }
}

// cpu.rs:249-257 for nt tokens at positions pos0+t: q heads (the first hd of each [q | gate]
// block of 2*hd) and k heads RMS-normed with their weights (nullptr = unit), then roped; q is
// rewritten in place, k_out receives the normed and roped k rows (f32, before the f16 cast of
// cpu.rs:258 which the caller applies).
//   q     : f32 q[t*q_tok_stride + h*2*hd + d]
//   k     : f32 k[t*kv_tok_stride + kh*hd + d]; k_out [t*nkv*hd + kh*hd + d]
void it_ref_attn_prep(float* q, int q_tok_stride, const float* k, int kv_tok_stride, const float* q_norm,
                      const float* k_norm, float eps, float* k_out, int pos0, int hd, int nh, int nkv, int nt,
                      int n_rot, float base, const int* sections) {
    std::vector<float> row(hd);
    for (int t = 0; t < nt; ++t) {
        for (int h = 0; h < nh; ++h) {
            float* qh = q + (size_t)t * q_tok_stride + (size_t)h * 2 * hd;
            it_ref_rmsnorm(qh, q_norm, hd, eps, row.data());
            it_ref_rope(row.data(), 1, hd, n_rot, pos0 + t, base, sections);
            std::memcpy(qh, row.data(), hd * sizeof(float));
        }
        for (int h = 0; h < nkv; ++h) {
            float* ko = k_out + ((size_t)t * nkv + h) * hd;
            it_ref_rmsnorm(k + (size_t)t * kv_tok_stride + (size_t)h * hd, k_norm, hd, eps, ko);
            it_ref_rope(ko, 1, hd, n_rot, pos0 + t, base, sections);
        }
    }
}

// cpu.rs:234-238 gated RMSNorm of the GDN output, per V head row of hv floats for nt tokens:
// out = rmsnorm(o_h, w, eps) * silu(z_h), rows at o[t*tok_stride + h*hv], z and out alike.
void it_ref_gdn_gated_norm(const float* o, const float* z, const float* w, int nv, int hv, int nt, int tok_stride,
                           float eps, float* out) {
    std::vector<float> n(hv);
    for (int t = 0; t < nt; ++t)
        for (int h = 0; h < nv; ++h) {
            const size_t b = (size_t)t * tok_stride + (size_t)h * hv;
            it_ref_rmsnorm(o + b, w, hv, eps, n.data());
            for (int j = 0; j < hv; ++j) out[b + j] = n[j] * silu(z[b + j]);
        }
}

// cpu.rs:164 l2norm, in place.
void it_ref_l2norm(float* x, int n, float eps) {
    float s = 0.0f; for (int i = 0; i < n; ++i) s += x[i] * x[i];
    float sc = 1.0f / std::max(std::sqrt(s), eps);
    for (int i = 0; i < n; ++i) x[i] *= sc;
}

// Softmax attention with sigmoid output gate over an f16 KV cache, cpu.rs:260-272, for nt query
// tokens. Token t attends to n = pos0 + t + 1 keys (the engine's causal convention: cpu.rs:260 with
// st.pos = pos0 + t, and the split-K kernels' n = pos0+t+1, kernels/src/lib.rs:764).
//   q    : f32, token t head h at q[t*q_tok_stride + h*2*hd] = q(hd) then gate(hd) (cpu.rs:249-254)
//   kc,vc: f16 bits [pos][kvd], kvd = nkv*hd; head kh at offset kh*hd (cpu.rs:259, 267, 270)
//   out  : f32 out[t*out_tok_stride + h*hd + j]
// The reference keeps K/V as f32 holding f16-rounded values in Numerics::Ggml (cpu.rs:258); here
// the cache is f16 and widened exactly, which is the same set of values.
}  // extern "C"

// The attention loop of cpu.rs:260-272 (and of the MTP head, src/mtp.rs:122-130), for either cache
// element type: the loader widens one cache element to f32.
template <class T, class Load>
static void attn_rows(const float* q, int q_tok_stride, const T* kc, const T* vc, int kvd, int pos0, int hd, int nh,
                      int nkv, int nt, float scale, float* out, int out_tok_stride, int threads, Load ld) {
    const int group = nh / nkv;
    par_for(nt * nh, threads, [&](int job) {
        const int t = job / nh, h = job % nh;
        const int kh = h / group;                                  // cpu.rs:265
        const int n = pos0 + t + 1;                                // cpu.rs:260
        const float* qh = q + (size_t)t * q_tok_stride + (size_t)h * 2 * hd;
        const float* gate = qh + hd;
        std::vector<float> sc(n);
        for (int p = 0; p < n; ++p) {                              // cpu.rs:267
            const T* kr = kc + (size_t)p * kvd + (size_t)kh * hd;
            float s = 0.0f;
            for (int i = 0; i < hd; ++i) s += qh[i] * ld(kr[i]);
            sc[p] = s * scale;
        }
        float mx = -INFINITY; for (int p = 0; p < n; ++p) mx = std::max(mx, sc[p]);   // cpu.rs:268
        float sum = 0.0f; for (int p = 0; p < n; ++p) { sc[p] = std::exp(sc[p] - mx); sum += sc[p]; } // :269
        float* oh = out + (size_t)t * out_tok_stride + (size_t)h * hd;
        for (int j = 0; j < hd; ++j) oh[j] = 0.0f;
        for (int p = 0; p < n; ++p) {                              // cpu.rs:270
            const float w = sc[p] / sum;
            const T* vr = vc + (size_t)p * kvd + (size_t)kh * hd;
            for (int j = 0; j < hd; ++j) oh[j] += w * ld(vr[j]);
        }
        for (int j = 0; j < hd; ++j) oh[j] *= sigmoid(gate[j]);   // cpu.rs:272
    });
}

extern "C" {

void it_ref_attn(const float* q, int q_tok_stride, const uint16_t* kc, const uint16_t* vc, int kvd,
                 int pos0, int hd, int nh, int nkv, int nt, float scale, float* out, int out_tok_stride,
                 int threads) {
    attn_rows(q, q_tok_stride, kc, vc, kvd, pos0, hd, nh, nkv, nt, scale, out, out_tok_stride, threads,
              [](uint16_t b) { return h2f(b); });
}

// The MTP head's attention over its f32 KV cache, src/mtp.rs:122-130: the same loop with f32 K/V.
// Slot p of the head's cache holds position p + 1 (mtp.rs:120); the caller passes pos0 = the first
// query's slot, so query t sees slots 0..pos0+t.
void it_ref_attn_f32kv(const float* q, int q_tok_stride, const float* kc, const float* vc, int kvd, int pos0, int hd,
                       int nh, int nkv, int nt, float scale, float* out, int out_tok_stride, int threads) {
    attn_rows(q, q_tok_stride, kc, vc, kvd, pos0, hd, nh, nkv, nt, scale, out, out_tok_stride, threads,
              [](float x) { return x; });
}

// Depthwise causal conv + SiLU with the rolling (K-1)-token state, oldest first, for nt tokens
// processed one after another (cpu.rs:201-212 once per forward_token call).
//   x    : f32 x[t*x_tok_stride + ch]  (the qkv matvec output "mixed")
//   w    : f32 w[ch*K + i]             (ssm_conv1d.weight, cpu.rs:207)
//   state: f32 state[i*cd + ch], i < K-1 (cpu.rs:131), updated in place
//   out  : f32 out[t*out_tok_stride + ch]
void it_ref_gdn_conv(const float* x, int x_tok_stride, const float* w, float* state, float* out,
                     int out_tok_stride, int cd, int nt, int K) {
    for (int t = 0; t < nt; ++t) {
        const float* mixed = x + (size_t)t * x_tok_stride;
        float* co = out + (size_t)t * out_tok_stride;
        for (int ch = 0; ch < cd; ++ch) {                         // cpu.rs:205-209
            float s = 0.0f;
            for (int i = 0; i < K; ++i) {
                float v = i < K - 1 ? state[(size_t)i * cd + ch] : mixed[ch];
                s += v * w[(size_t)ch * K + i];
            }
            co[ch] = silu(s);
        }
        for (int i = 0; i + 2 < K; ++i)                           // cpu.rs:211
            for (int ch = 0; ch < cd; ++ch) state[(size_t)i * cd + ch] = state[(size_t)(i + 1) * cd + ch];
        for (int ch = 0; ch < cd; ++ch) state[(size_t)(K - 2) * cd + ch] = mixed[ch];   // cpu.rs:212
    }
}

// Gated-delta recurrence for nt tokens, each as one forward_token step (cpu.rs:213-232), after the
// conv output `co` has been L2-normalised on its 2*nk q/k heads (cpu.rs:214; call it_ref_l2norm).
//   co   : f32 co[t*co_tok_stride + c]: q heads [0, nk*S), k heads [nk*S, 2nk*S), v heads [2nk*S, ..)
//   beta_raw, alpha_raw: f32 [t*ba_tok_stride + h] (matvec outputs b_raw, al; cpu.rs:199-200)
//   dt, a: f32 [nv] (ssm_dt.bias, ssm_a; cpu.rs:222)
//   state: f32, layout [h][i][j] = S[i][j] with i the key index and j the value index. (The
//          reference CPU stores M[j][i] = S[i][j], cpu.rs:132; the GPU arena stores T[i*S+j],
//          shaders/gdn.comp:2. This oracle uses the GPU layout so both sides share one buffer
//          format; the arithmetic below is the cpu.rs loop order with the index swapped.)
//   out  : f32 out[t*out_tok_stride + h*S + j]
void it_ref_gdn_step(const float* co, int co_tok_stride, const float* beta_raw, const float* alpha_raw,
                     int ba_tok_stride, const float* dt, const float* a, float* state, float* out,
                     int out_tok_stride, int nt, int nv, int nk, int S, int threads) {
    const int qk = nk * S;
    const float scale = 1.0f / std::sqrt((float)S);              // cpu.rs:215
    par_for(nv, threads, [&](int h) {
        std::vector<float> col(S);
        float* m = state + (size_t)h * S * S;
        for (int t = 0; t < nt; ++t) {
            const float* c = co + (size_t)t * co_tok_stride;
            const int kh = h % nk;                                 // cpu.rs:219
            const float* q = c + (size_t)kh * S;
            const float* k = c + qk + (size_t)kh * S;
            const float* v = c + 2 * qk + (size_t)h * S;
            const float bt = sigmoid(beta_raw[(size_t)t * ba_tok_stride + h]);                  // cpu.rs:222
            const float g = softplus(alpha_raw[(size_t)t * ba_tok_stride + h] + dt[h]) * a[h];
            const float eg = std::exp(g);
            float* oh = out + (size_t)t * out_tok_stride + (size_t)h * S;
            for (int j = 0; j < S; ++j) {                          // cpu.rs:223-231, row j of M
                for (int i = 0; i < S; ++i) col[i] = m[(size_t)i * S + j];
                float s = 0.0f;
                for (int i = 0; i < S; ++i) { col[i] *= eg; s += col[i] * k[i]; }
                const float delta = (v[j] - s) * bt;
                float acc = 0.0f;
                for (int i = 0; i < S; ++i) { col[i] += k[i] * delta; acc += col[i] * q[i]; }
                oh[j] = acc * scale;
                for (int i = 0; i < S; ++i) m[(size_t)i * S + j] = col[i];
            }
        }
    });
}

// One full GDN token pass as cpu.rs:201-232 does it: conv (+state shift) -> L2 on the 2*nk q/k
// heads -> recurrence, token after token. `co_scratch` receives the normalised conv output
// [nt][cd]. eps is the model's rms epsilon (cpu.rs:214).
void it_ref_gdn_layer(const float* x, int x_tok_stride, const float* w, float* conv_state, int K,
                      const float* beta_raw, const float* alpha_raw, int ba_tok_stride,
                      const float* dt, const float* a, float* state, float* out, int out_tok_stride,
                      float* co_scratch, int nt, int nv, int nk, int S, float eps, int threads) {
    const int cd = 2 * nk * S + nv * S;                           // model.rs:41-42
    for (int t = 0; t < nt; ++t) {
        float* co = co_scratch + (size_t)t * cd;
        it_ref_gdn_conv(x + (size_t)t * x_tok_stride, x_tok_stride, w, conv_state, co, cd, cd, 1, K);
        for (int h = 0; h < 2 * nk; ++h) it_ref_l2norm(co + (size_t)h * S, S, eps);
        it_ref_gdn_step(co, cd, beta_raw + (size_t)t * ba_tok_stride, alpha_raw + (size_t)t * ba_tok_stride,
                        ba_tok_stride, dt, a, state, out + (size_t)t * out_tok_stride, out_tok_stride,
                        1, nv, nk, S, threads);
    }
}

} // extern "C"
