/* Sweeps it_attn_plan over every decode / verify / chunk geometry a reference engine can issue at a
 * given context capacity and checks that the chosen records fit the reference's arena room
 * (attention_dispatch_room, src/vk/mod.rs:148-150, in words). Host-only: loads libit_attn.so with
 * dlopen and calls no device function. Prints "ok <plans>" or the first failing geometry.
 * With a sixth argument "f32kv" it sweeps it_attn_f32kv_plan (the MTP head's attention) instead,
 * with the room of the configured capacity divided by an optional seventh argument (default 1),
 * and prints "ok <plans> <grown> <one_pass>". */
#include <dlfcn.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef int (*plan_fn)(int, int, int, int, int, size_t, int*, int*, size_t*);
typedef size_t (*room_fn)(size_t, size_t, size_t);
typedef int (*plan32_fn)(int, int, int, int, int, size_t, int*, size_t*);

/* every f32-KV plan fits the room, splits are multiples of 64 keys, the preferred split is kept when
 * it fits and the one-pass form is used only where one record per (token, head) does not fit */
static int sweep_f32kv(void* h, int nh, int nkv, int ctxmax, int ntmax, int div) {
    plan32_fn plan = (plan32_fn)dlsym(h, "it_attn_f32kv_plan");
    room_fn room = (room_fn)dlsym(h, "it_attention_dispatch_room");
    if (!plan || !room) { fprintf(stderr, "missing symbols\n"); return 2; }
    long plans = 0, grown = 0, one_pass = 0;
    for (int nt = 1; nt <= ntmax; ++nt) {
        const size_t budget = room(ctxmax, nh, nt) * 4 / div;
        for (int pos0 = 0; pos0 + nt <= ctxmax; ++pos0) {
            int chunk = -1, c2 = -1;
            size_t bytes = 0, pref = 0;
            if (plan(pos0, nt, 256, nh, nkv, budget, &chunk, &bytes) != 0 || bytes > budget || chunk < 0 ||
                chunk % 64 != 0) {
                printf("FAIL nt=%d pos0=%d budget=%zu chunk=%d bytes=%zu\n", nt, pos0, budget, chunk, bytes);
                return 1;
            }
            const size_t one_rec = (size_t)nt * nh * 260 * 4;
            if (chunk == 0 && one_rec <= budget) {
                printf("FAIL one pass although a record per row fits nt=%d pos0=%d\n", nt, pos0);
                return 1;
            }
            if (chunk && bytes != (size_t)nt * nh * ((pos0 + nt + chunk - 1) / chunk) * 260 * 4) {
                printf("FAIL bytes formula nt=%d pos0=%d chunk=%d\n", nt, pos0, chunk);
                return 1;
            }
            plan(pos0, nt, 256, nh, nkv, (size_t)-1, &c2, &pref);
            if (pref <= budget && (c2 != chunk || pref != bytes)) {
                printf("FAIL preferred split not kept nt=%d pos0=%d\n", nt, pos0);
                return 1;
            }
            if (chunk != c2) ++grown;
            if (chunk == 0) ++one_pass;
            ++plans;
        }
    }
    printf("ok %ld %ld %ld\n", plans, grown, one_pass);
    return 0;
}

int main(int argc, char** argv) {
    if (argc < 6) { fprintf(stderr, "usage: plan_sweep LIB NH NKV CTXMAX NTMAX\n"); return 2; }
    void* h = dlopen(argv[1], RTLD_NOW);
    if (!h) { fprintf(stderr, "dlopen: %s\n", dlerror()); return 2; }
    plan_fn plan = (plan_fn)dlsym(h, "it_attn_plan");
    room_fn room = (room_fn)dlsym(h, "it_attention_dispatch_room");
    if (!plan || !room) { fprintf(stderr, "missing symbols\n"); return 2; }
    const int nh = atoi(argv[2]), nkv = atoi(argv[3]), ctxmax = atoi(argv[4]), ntmax = atoi(argv[5]);
    if (argc > 6 && !strcmp(argv[6], "f32kv")) return sweep_f32kv(h, nh, nkv, ctxmax, ntmax, argc > 7 ? atoi(argv[7]) : 1);
    long plans = 0, flash_one_pass = 0, grown = 0;
    for (int nt = 1; nt <= ntmax; ++nt) {
        for (int pos0 = 0; pos0 + nt <= ctxmax; ++pos0) {
            /* the engine's capacity is at least pos0 + nt: test the tightest and the configured one */
            const int caps[2] = {pos0 + nt, ctxmax};
            for (int ci = 0; ci < 2; ++ci) {
                if (ci == 1 && caps[1] == caps[0]) continue;
                const size_t budget = room(caps[ci], nh, nt) * 4;
                int kernel = -1, chunk = -1;
                size_t bytes = 0, pref = 0;
                if (plan(pos0, nt, 256, nh, nkv, budget, &kernel, &chunk, &bytes) != 0 || bytes > budget) {
                    printf("FAIL nt=%d pos0=%d ctx=%d budget=%zu kernel=%d chunk=%d bytes=%zu\n", nt, pos0, caps[ci],
                           budget, kernel, chunk, bytes);
                    return 1;
                }
                /* with an unlimited budget the plan is the library's preferred one */
                int k2, c2;
                plan(pos0, nt, 256, nh, nkv, (size_t)-1, &k2, &c2, &pref);
                if (k2 != kernel) { printf("FAIL kernel changed nt=%d pos0=%d\n", nt, pos0); return 1; }
                if (bytes < pref) ++grown;
                if (kernel == 2 && chunk == 0) ++flash_one_pass;
                ++plans;
            }
        }
    }
    printf("ok %ld %ld %ld\n", plans, grown, flash_one_pass);
    return 0;
}
