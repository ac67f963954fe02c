"""The C-ABI library loads, exports every symbol include/it_attn.h declares, and its host-side
policy / validation behaves like the reference's (no device work in these tests)."""
import ctypes
import os
import re

import pytest

from irontimber_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_symbols():
    text = open(os.path.join(ROOT, "include", "it_attn.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(it_[a-z0-9_]+)\s*\(", text)))


def test_header_symbols_exported_and_bound():
    lib = _lib.lib()
    syms = header_symbols()
    assert len(syms) >= 15
    for s in syms:
        assert hasattr(lib, s), s
        assert s in _lib.SIGNATURES, f"{s} missing from the ctypes binding"


def test_abi_version():
    assert _lib.lib().it_abi_version() == 1


def test_scratch_words_and_room_match_reference():
    """prefill_review.rs:18, 27: attention_scratch_words / attention_dispatch_room."""
    lib = _lib.lib()
    assert lib.it_attention_scratch_words(8192, 24) == 64 * 8192 * 24
    assert lib.it_attention_scratch_words(16, 24) == 64 * 260 * 24
    for nt in [1, 2, 22, 43, 64, 128, 256, 512]:
        assert lib.it_attention_dispatch_room(8192, 24, nt) == (nt + 63) // 64 * 64 * 8192 * 24
    assert lib.it_attention_dispatch_room(8192, 24, 0) == 0
    assert lib.it_attention_dispatch_room(8192, 24, 513) == 0


@pytest.mark.parametrize("ctx", [1, 16, 192, 256, 260, 8192])
def test_chunk_policy_fits_room(ctx):
    """prefill_review.rs:35-40: for nt = min(ctx,64) the chosen C keeps the partials in the room."""
    lib = _lib.lib()
    room = lib.it_attention_scratch_words(ctx, 24)
    nt = min(ctx, 64)
    c = lib.it_attention_chunk(nt, 24, ctx - nt, room)
    assert c in (64, 128, 256, 512, 1024)
    assert nt * 24 * ((ctx + c - 1) // c) * 260 <= room


def test_chunk_policy_decode_is_64():
    lib = _lib.lib()
    room = lib.it_attention_dispatch_room(8192, 16, 1)
    assert lib.it_attention_chunk(1, 16, 8191, room) == 64


def test_validate_geometry():
    """r012_review.rs:6-7: production geometry passes, each broken field fails, ctx 0/8193 fail."""
    lib = _lib.lib()
    ok = dict(ctx_len=8192, head_dim=256, n_head=16, n_head_kv=2, ssm_state=128, ssm_groups=16,
              ssm_vheads=32, ssm_inner=4096, conv_k=4)
    assert lib.it_validate_geometry(*ok.values()) == 0
    for k, bad in [("head_dim", 128), ("n_head_kv", 0), ("conv_k", 5), ("ssm_state", 64), ("ssm_groups", 0),
                   ("ctx_len", 0), ("ctx_len", 8193), ("n_head", 15), ("ssm_inner", 4000)]:
        g = dict(ok, **{k: bad})
        assert lib.it_validate_geometry(*g.values()) != 0, k
        assert _lib.last_error()


def test_attn_rejects_bad_geometry_before_device_work():
    """Validation fails before any launch (the MUST_NOT_QUERY_DEVICE sentinels of prefill_review.rs:42)."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced: validation must fail first
    rc = lib.it_attn_f16(fake, 512, fake, fake, 256, 0, 128, 1, 1, 1, 0.1, fake, 128, None, 0, None)
    assert rc != 0 and "head_dim" in _lib.last_error()
    rc = lib.it_attn_f16(fake, 8192, fake, fake, 512, 0, 256, 15, 2, 1, 0.1, fake, 4096, None, 0, None)
    assert rc != 0 and "n_head" in _lib.last_error()
    rc = lib.it_attn_f16_ex(fake, 8192, fake, fake, 512, 0, 256, 16, 2, 1, 0.1, fake, 4096, None, 0, 1, 64, None)
    assert rc != 0 and "scratch" in _lib.last_error()
    rc = lib.it_attn_f16_ex(fake, 8192, fake, fake, 512, 0, 256, 16, 2, 4, 0.1, fake, 4096, fake, 1 << 30, 2, 96, None)
    assert rc != 0 and "multiple of 64" in _lib.last_error()
    rc = lib.it_gdn_step(fake, 8192, fake, fake, 32, fake, fake, fake, fake, 4096, 1, 32, 16, 64, None)
    assert rc != 0 and "state size" in _lib.last_error()
    rc = lib.it_gdn_conv(fake, 8192, fake, fake, fake, 8192, 8192, 1, 5, None)
    assert rc != 0 and "kernel size" in _lib.last_error()
    rc = lib.it_kv_append_f16(fake, fake, 512, fake, fake, 0, 1, 512, 2, None)
    assert rc != 0 and "round_mode" in _lib.last_error()
    # fused GDN decode layer: token count, and the conv-state buffers must not overlap
    rc = lib.it_gdn_decode_fused(fake, 8192, fake, 4, fake, fake, fake, fake, 32, fake, fake, fake, fake, 4096, 5,
                                 32, 16, 128, 1e-6, None)
    assert rc != 0 and "nt 5" in _lib.last_error()
    st_in, st_out = ctypes.c_void_p(1 << 20), ctypes.c_void_p((1 << 20) + 4096)
    rc = lib.it_gdn_decode_fused(fake, 8192, fake, 4, st_in, st_out, fake, fake, 32, fake, fake, fake, fake, 4096, 1,
                                 32, 16, 128, 1e-6, None)
    assert rc != 0 and "overlaps" in _lib.last_error()
    # checkpointed form: ck_after inside the batch, checkpoint buffers apart from the states
    st_in2 = ctypes.c_void_p(1 << 24)
    rc = lib.it_gdn_decode_fused_ckpt(fake, 8192, fake, 4, st_in2, st_out, fake, fake, 32, fake, fake, fake, fake, 4096,
                                      2, 32, 16, 128, 1e-6, ctypes.c_void_p(1 << 28), ctypes.c_void_p(1 << 29), 2, None)
    assert rc != 0 and "checkpoint token 2" in _lib.last_error()
    rc = lib.it_gdn_decode_fused_ckpt(fake, 8192, fake, 4, st_in2, st_out, fake, fake, 32, fake, fake, fake, fake, 4096,
                                      2, 32, 16, 128, 1e-6, ctypes.c_void_p(1 << 28), st_out, 0, None)
    assert rc != 0 and "overlaps" in _lib.last_error()



def test_q16_entries_reject_bad_arguments_before_device_work():
    """it_attn_prep_f16_q16 / it_attn_f16_q16: a missing, misaligned or overlapping q16, or a bad
    scale, fails before any launch, as do the checks the plain calls make."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(1 << 20)

    def attn(q16=fake, q16ts=4096, hd=256, nt=64):
        return lib.it_attn_f16_q16(fake, 8192, q16, q16ts, fake, fake, 512, 0, hd, 16, 2, nt, 0.0625, fake, 4096, None,
                                   0, None)
    assert attn(q16=None) != 0 and "q16" in _lib.last_error()
    assert attn(q16=ctypes.c_void_p((1 << 20) + 8)) != 0 and "16-byte" in _lib.last_error()
    assert attn(q16ts=4092) != 0 and "multiple of 8" in _lib.last_error()
    assert attn(q16ts=2048) != 0 and "overlaps" in _lib.last_error()
    assert attn(hd=128) != 0 and "head_dim" in _lib.last_error()

    def prep(q16=fake, q16ts=4096, scale=0.0625, rm=0):
        return lib.it_attn_prep_f16_q16(fake, 8192, fake, fake, 512, None, None, 1e-6, fake, fake, 512, 0, 256, 16, 2,
                                        64, 64, 0.5, 0, 0, 0, 0, rm, q16, q16ts, scale, None)
    assert prep(q16=None) != 0 and "q16" in _lib.last_error()
    assert prep(q16ts=4092) != 0 and "multiple of 8" in _lib.last_error()
    assert prep(q16ts=2048) != 0 and "overlaps" in _lib.last_error()
    assert prep(scale=0.0) != 0 and "scale" in _lib.last_error()
    assert prep(rm=2) != 0 and "round_mode" in _lib.last_error()

def test_record_layout_entries_reject_bad_arguments_before_device_work():
    """it_attn_partials_ex / it_attn_combine_ex: an unknown layout, or the piece layout (1) for a
    geometry whose merge is not the wave merge (at most 16 splits, or more than 256 rows), fails
    before any launch."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(1 << 20)
    big = 1 << 30

    def part(layout, pos0=8191, nt=1, chunk=64):
        return lib.it_attn_partials_ex(fake, 8192, fake, fake, 512, pos0, 256, 16, 2, nt, 0.0625, fake, big, chunk,
                                       layout, None)

    def comb(layout, pos0=8191, nt=1, chunk=64):
        return lib.it_attn_combine_ex(fake, 8192, fake, pos0, 256, 16, nt, chunk, layout, fake, 4096, None)
    for f in (part, comb):
        assert f(2) != 0 and "layout" in _lib.last_error()
        assert f(1, pos0=511) != 0 and "9-256 splits" in _lib.last_error()       # 8 splits
        assert f(1, pos0=8192 * 4) != 0 and "9-256 splits" in _lib.last_error()  # 513 splits
        assert f(1, pos0=8128, nt=64) != 0 and "256" in _lib.last_error()         # 1024 rows
        assert f(1, chunk=96) != 0 and "multiple of 64" in _lib.last_error()


def test_short_context_split_policy():
    """Split-K plans below 2048 keys: 32-key splits for 1-2 tokens (more workgroups), except where
    the one-launch mailbox form could launch (at most 8 query rows per KV head and at most 4 merge
    units per workgroup with 64-key splits), which must stay bit-equal to it_attn_f16; 4-token calls
    and contexts from 2048 keys keep 64-key splits."""
    lib = _lib.lib()

    def plan(pos0, nt, nh=16, nkv=2):
        k, c, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
        assert lib.it_attn_plan(pos0, nt, 256, nh, nkv, ctypes.c_size_t(1 << 40), ctypes.byref(k), ctypes.byref(c),
                                ctypes.byref(b)) == 0
        return k.value, c.value
    assert plan(511, 1) == (1, 32) and plan(1983, 1) == (1, 32) and plan(62, 2) == (1, 32)
    assert plan(2046, 2) == (1, 64) and plan(8191, 1) == (1, 64)
    assert plan(1020, 4) == (1, 64)
    # 2000 keys: 32 splits x 2 KV heads of 64 keys give 64 workgroups for 256 merge units, so the
    # mailbox could launch: 64 keys (also with 32 heads over 4 KV heads)
    assert plan(1999, 1) == (1, 64) and plan(1999, 1, 32, 4) == (1, 64)
    # explicit splits: multiples of 32 for the split-K kernel
    assert lib.it_attn_scratch_bytes_ex(511, 1, 256, 16, 2, 1, 32) == 16 * 16 * 260 * 4


def test_scratch_bytes_policy():
    lib = _lib.lib()
    # decode: split-K, C = 64 -> 128 splits of 260 words per head
    assert lib.it_attn_scratch_bytes(8191, 1, 256, 16, 2) == 16 * 128 * 260 * 4
    # MTP verify (32 rows per KV head): C = 64
    assert lib.it_attn_scratch_bytes(8188, 4, 256, 16, 2) == 4 * 16 * 128 * 260 * 4
    # whole-prompt prefill: flash, no scratch
    assert lib.it_attn_scratch_bytes(0, 8192, 256, 16, 2) == 0
    # a 64-token chunk after 4096 positions: 8 flash row tiles, keys split 192 per split (22
    # splits); the flash kernel's records are 132 words (16-byte header, 256 int16)
    assert lib.it_attn_scratch_bytes(4096, 64, 256, 16, 2) == 64 * 16 * 22 * 132 * 4
    # forced one-pass flash (chunk >= keys) and forced splits
    assert lib.it_attn_scratch_bytes_ex(4096, 64, 256, 16, 2, 2, 8192) == 0
    assert lib.it_attn_scratch_bytes_ex(4096, 64, 256, 16, 2, 2, 1024) == 64 * 16 * 5 * 132 * 4


@pytest.mark.parametrize("nh,nkv", [(16, 2), (24, 4)])
def test_plan_fits_reference_room_sweep(tmp_path, nh, nkv):
    """Every (nt 1..512, pos0 <= 8192-nt) with the engine's capacity at pos0+nt and at 8192: the
    split it_attn_f16 picks fits attention_dispatch_room words (src/vk/mod.rs:148-150, 714-716)."""
    import subprocess
    exe = tmp_path / "plan_sweep"
    subprocess.run(["gcc", "-O2", "-o", str(exe), os.path.join(ROOT, "tests", "csrc", "plan_sweep.c"), "-ldl"],
                   check=True)
    r = subprocess.run([str(exe), _lib.LIB_PATH, str(nh), str(nkv), "8192", "512"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr
    plans, grown, _ = map(int, r.stdout.split()[1:])
    assert plans == 8126464 and grown > 0


def plan(pos0, nt, nh, nkv, budget):
    k, c, b = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
    rc = _lib.lib().it_attn_plan(pos0, nt, 256, nh, nkv, budget, ctypes.byref(k), ctypes.byref(c), ctypes.byref(b))
    return rc, k.value, c.value, b.value


def test_plan_config3_positions_fit_reference_room():
    """The config-3 chunk positions that overflowed the room with the preferred split now grow it."""
    lib = _lib.lib()
    room = lib.it_attention_dispatch_room(8192, 16, 64) * 4
    for pos0 in (3968, 4032, 5952, 6016, 6080, 7936, 8000, 8064, 8128):
        pref = lib.it_attn_scratch_bytes(pos0, 64, 256, 16, 2)
        rc, k, c, b = plan(pos0, 64, 16, 2, room)
        assert rc == 0 and k == 2 and b <= room
        assert pref > room or b == pref
        assert c == 0 or c % 64 == 0


def test_plan_decode_keeps_64_and_small_budget_fails_cleanly():
    lib = _lib.lib()
    room = lib.it_attention_dispatch_room(8192, 16, 1) * 4
    assert plan(8191, 1, 16, 2, room)[1:3] == (1, 64)
    # one record per (token, head) is the floor of the split-K kernel
    rc, k, c, b = plan(8191, 1, 16, 2, 16 * 1040 - 1)
    assert rc != 0 and "one record" in _lib.last_error()
    assert plan(8191, 1, 16, 2, 16 * 1040)[0] == 0
    # the flash kernel always has a plan: one pass needs no scratch
    assert plan(4096, 64, 16, 2, 0)[1:] == (2, 0, 0)


def prefill_chunks(n, batch):
    lib = _lib.lib()
    cnt = lib.it_prefill_chunks(n, batch, None, None, 0)
    if cnt < 0:
        return None
    st, ln = (ctypes.c_size_t * max(cnt, 1))(), (ctypes.c_size_t * max(cnt, 1))()
    assert lib.it_prefill_chunks(n, batch, st, ln, cnt) == cnt
    return [(st[i], st[i] + ln[i]) for i in range(cnt)]


def test_prefill_chunks_cover_every_token():
    """prefill_review.rs:20-25: every range non-empty and <= batch, ids 0..n in order, 129 @ 512."""
    for batch in (64, 128, 256, 512):
        for n in (0, 1, 21, 22, 64, 65, 129, 2091, 4191, 7416, 8192):
            rr = prefill_chunks(n, batch)
            ids = []
            for a, b in rr:
                assert 0 < b - a <= batch
                ids.extend(range(a, b))
            assert ids == list(range(n))
    assert prefill_chunks(129, 512) == [(0, 128), (128, 129)]
    assert prefill_chunks(8192, 64) == [(64 * i, 64 * i + 64) for i in range(128)]
    # a tail of 22 or more tokens stays in its range; 1..21 past a multiple of 64 is peeled
    assert prefill_chunks(150, 512) == [(0, 150)]
    assert prefill_chunks(148, 512) == [(0, 128), (128, 148)]
    assert prefill_chunks(85, 128) == [(0, 64), (64, 85)]
    assert prefill_chunks(86, 128) == [(0, 86)]
    assert prefill_chunks(70, 64) == [(0, 64), (64, 70)]
    for bad in (0, 32, 65, 1024):
        assert prefill_chunks(100, bad) is None and "unsupported prefill batch" in _lib.last_error()


def test_prefill_chunks_brute_force():
    """Against a direct statement of the rule for every n <= 1100 and every batch."""
    for batch in (64, 128, 256, 512):
        for n in range(0, 1100):
            want, s = [], 0
            while s < n:
                m = min(n - s, batch)
                if m > 64 and 0 < m % 64 < 22:
                    m -= m % 64
                want.append((s, s + m))
                s += m
            assert prefill_chunks(n, batch) == want


def test_mailbox_host_side():
    """The mailbox entry points' host-side rules, with no device work: the size formula (64 header
    words, then 96-byte pieces per token, head, 16-dim block and 64-key split), argument checks of
    the initialiser and the call before any launch, and the eligibility query declining every
    geometry that is not a decode step (no device query for those)."""
    lib = _lib.lib()
    for ctx, nt, nh in [(1, 1, 16), (8192, 1, 16), (8192, 4, 16), (16384, 1, 32), (65, 2, 8)]:
        smax = (ctx + 63) // 64
        assert lib.it_attn_mailbox_bytes(ctx, nt, nh) == 4 * (64 + nt * nh * 16 * smax * 24)
    assert lib.it_attn_mailbox_bytes(0, 1, 16) == 0 and lib.it_attn_mailbox_bytes(8192, 0, 16) == 0
    fake = ctypes.c_void_p(1 << 20)   # never dereferenced
    assert lib.it_attn_mailbox_init(None, 1 << 20, None) != 0
    assert lib.it_attn_mailbox_init(fake, 16, None) != 0                       # below one header
    assert lib.it_attn_mailbox_init(ctypes.c_void_p((1 << 20) + 4), 1 << 20, None) != 0   # misaligned
    assert b"16-byte" in lib.it_last_error()
    assert lib.it_attn_mailbox_poisoned(None, None, None) != 0
    # misaligned mailbox: refused before any device work
    rc = lib.it_attn_f16_mailbox(fake, 8192, fake, fake, 512, 8191, 256, 16, 2, 1, 0.0625, fake, 4096,
                                 ctypes.c_void_p((1 << 20) + 8), 1 << 22, None, 0, None)
    assert rc != 0 and b"16-byte" in lib.it_last_error()
    # bad geometry: the same validation as it_attn_f16
    rc = lib.it_attn_f16_mailbox(fake, 8192, fake, fake, 512, 0, 256, 15, 2, 1, 0.0625, fake, 4096, fake, 1 << 22,
                                 None, 0, None)
    assert rc != 0
    # not a decode step, too many splits, too small a mailbox, bad geometry: declined without a query
    need = lib.it_attn_mailbox_bytes(8192, 1, 16)
    assert lib.it_attn_mailbox_would_launch(8128, 64, 256, 16, 2, 1 << 30) == 0
    assert lib.it_attn_mailbox_would_launch(8191, 4, 256, 16, 2, 1 << 30) == 0      # 32 rows per KV head
    assert lib.it_attn_mailbox_would_launch(16384, 1, 256, 16, 2, 1 << 30) == 0     # 257 splits
    assert lib.it_attn_mailbox_would_launch(8191, 1, 256, 16, 2, need - 4) == 0
    assert lib.it_attn_mailbox_would_launch(8191, 1, 128, 16, 2, need) == 0


def test_gdn_prefill_host_side():
    """it_gdn_prefill: scratch size = f16 conv output (256-byte rounded) + the chunk records, and
    every argument error reported before device work. A record per (64-token chunk, V head) holds
    Kh^T (f16, 16 KiB), P (f16, 8 KiB) and the 1 KiB decay table; from an f32 conv output
    (it_gdn_chunked) also the chunk's q and k rows as f16 (2 x 16 KiB), which it_gdn_prefill's
    scan reads from its f16 conv output instead."""
    lib = _lib.lib()
    for nt, nv, nk in [(1, 32, 16), (64, 4, 2), (8192, 32, 16), (77, 8, 8)]:
        co = (nt * (2 * nk + nv) * 128 * 2 + 255) // 256 * 256
        nch = (nt + 63) // 64
        assert lib.it_gdn_prefill_scratch_bytes(nt, nv, nk, 128) == co + nch * nv * 25 * 1024
        assert lib.it_gdn_chunked_scratch_bytes(nt, nv, 128) == nch * nv * 57 * 1024
    assert lib.it_gdn_prefill_scratch_bytes(0, 32, 16, 128) == 0 and lib.it_gdn_prefill_scratch_bytes(8, 32, 16, 64) == 0
    fake = ctypes.c_void_p(1 << 20)
    need = lib.it_gdn_prefill_scratch_bytes(64, 32, 16, 128)

    def call(K=4, S=128, nv=32, nk=16, nt=64, scratch=fake, nbytes=need, xts=8192, ots=4096):
        return lib.it_gdn_prefill(fake, xts, fake, K, fake, fake, fake, nv, fake, fake, fake, fake, ots, nt, nv, nk, S,
                                  1e-6, scratch, nbytes, None)
    assert call(K=5) != 0
    assert call(S=64) != 0
    assert call(nv=30) != 0                       # nv not a multiple of nk
    assert call(xts=4096) != 0                    # token stride below cd = 8192
    assert call(ots=4098) != 0                    # out stride not a multiple of 4
    assert call(nbytes=need - 16) != 0 and b"scratch" in lib.it_last_error()
    assert call(scratch=ctypes.c_void_p((1 << 20) + 8)) != 0 and b"16-byte" in lib.it_last_error()
    assert call(nt=0) == 0                        # nothing to do, no device work


@pytest.mark.parametrize("nh,nkv,ctx,div", [(16, 2, 8192, 1), (24, 4, 8192, 1), (16, 2, 300, 1), (16, 2, 8192, 16),
                                            (24, 4, 8192, 64), (16, 2, 8192, 4096)])
def test_f32kv_plan_fits_reference_room_sweep(nh, nkv, ctx, div):
    """The MTP head's f32-KV attention: for every nt 1..64 and pos0 <= ctx - nt, the split that
    it_attn_f32kv picks for the reference room at capacity ctx (attention_dispatch_room,
    src/vk/mod.rs:148-150), or for 1/div of it, fits it, keeps the preferred split when that fits,
    follows the record formula, and takes the one-pass form only where a record per (token, head)
    does not fit."""
    import subprocess
    exe = os.path.join(ROOT, "tests", "csrc", "plan_sweep")
    r = subprocess.run([exe, _lib.LIB_PATH, str(nh), str(nkv), str(ctx), "64", "f32kv", str(div)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr
    plans, grown, one_pass = map(int, r.stdout.split()[1:])
    assert plans == sum(ctx - nt + 1 for nt in range(1, 65))
    # the one-pass form exactly for the call sizes whose one record per (token, head) exceeds the
    # budget (every pos0 of such an nt)
    room = lambda nt: _lib.lib().it_attention_dispatch_room(ctx, nh, nt) * 4 // div
    assert one_pass == sum(ctx - nt + 1 for nt in range(1, 65) if nt * nh * 1040 > room(nt))
    if div == 1 and ctx == 8192:   # the reference room holds the preferred split everywhere
        assert grown == 0 and one_pass == 0
    if div > 1:   # a smaller arena: splits grow
        assert grown > 0


def f32kv_plan(pos0, nt, nh, nkv, budget):
    c, b = ctypes.c_int(), ctypes.c_size_t()
    rc = _lib.lib().it_attn_f32kv_plan(pos0, nt, 256, nh, nkv, budget, ctypes.byref(c), ctypes.byref(b))
    return rc, c.value, b.value


def test_f32kv_plan_cases():
    lib = _lib.lib()
    # decode at 8192 slots keeps 64-key splits within the room
    room1 = lib.it_attention_dispatch_room(8192, 16, 1) * 4
    assert f32kv_plan(8191, 1, 16, 2, room1) == (0, 64, 16 * 128 * 1040)
    # the MTP catch-up of 64 tokens at slot 4096: 64-key splits would need 69,222,400 B against a
    # room of 33,554,432 B (the reference doubles its C from 64 to 256 to fit, src/vk/mod.rs:731-733);
    # the library's split for multi-block calls minimises rounds of workgroups over the 256 CUs x
    # (tiles + 1): at slot 4096, 576 keys (8 splits x 2 KV heads x 16 row blocks = 256 workgroups,
    # one round of 9 tiles), 8,519,680 B, inside the room
    room64 = lib.it_attention_dispatch_room(8192, 16, 64) * 4
    assert room64 == 33554432
    assert 64 * 16 * 65 * 1040 == 69222400
    total, c = 4096 + 64, 64
    while c < 1024 and 64 * 16 * -(-total // c) * 260 * 4 > room64:
        c *= 2
    assert c == 256
    assert lib.it_attn_f32kv_scratch_bytes(4096, 64, 256, 16, 2) == 64 * 16 * 8 * 1040
    assert f32kv_plan(4096, 64, 16, 2, room64) == (0, 576, 64 * 16 * 8 * 1040)
    # the cost model by hand: rounds x (tiles + 1) for every candidate, ties to the longer split
    def cost(c, total=4160, per_split=2 * 16):
        return -(-(-(-total // c) * per_split) // 256) * (c // 64 + 1)
    costs = {c: cost(c) for c in range(64, 4160 + 64, 64)}
    best = min(costs.values())
    assert max(c for c, v in costs.items() if v == best) == 576 and costs[256] == 15 and costs[576] == 10
    # at slot 8128, 1024 keys (8 splits: 256 workgroups, one round of 16 tiles); a budget of 5
    # records per row doubles it to 2048
    assert f32kv_plan(8128, 64, 16, 2, room64) == (0, 1024, 64 * 16 * 8 * 1040)
    assert f32kv_plan(8128, 64, 16, 2, 64 * 16 * 5 * 1040) == (0, 2048, 64 * 16 * 4 * 1040)
    # one row block (decode, verify) keeps 64-key splits
    assert f32kv_plan(8188, 4, 16, 2, 1 << 40)[1] == 64
    # past the reference's 1024 keys: one split over every key still needs only a record per row
    assert f32kv_plan(8000, 64, 16, 2, 64 * 16 * 1040) == (0, 8192, 64 * 16 * 1040)
    # below one record per (token, head): the one-pass form, no scratch
    assert f32kv_plan(8000, 64, 16, 2, 64 * 16 * 1040 - 1) == (0, 0, 0)
    assert f32kv_plan(10, 1, 16, 2, 0) == (0, 0, 0)
    # bad geometry
    assert f32kv_plan(10, 1, 16, 3, 0)[0] != 0 and "bad geometry" in _lib.last_error()
    assert f32kv_plan(10, 1, 34, 2, 0)[0] != 0
