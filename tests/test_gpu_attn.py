"""GPU parity of the attention path (C ABI through irontimber_amd.ops) against the oracle."""
import numpy as np
import pytest
import torch

import oracle
from oracle.ref_np import attn_f64, f16_to_f64
from irontimber_amd import ops
from irontimber_amd.synth import attn_inputs, f16_bits, f16_bits_rtz
from tests.gpu_util import announce, assert_argmax_agrees, dev_f16bits, dev_f32, host
from tests.r012 import CASES, GEOMS, arena

pytestmark = pytest.mark.gpu
TOL = 2e-3   # max abs error on attention outputs


def run_case(dev, seed, ctx, nt, nh=16, nkv=2, kernel=ops.KERNEL_AUTO, chunk=0):
    pos0 = ctx - nt
    q, kb, vb = attn_inputs(seed, ctx=ctx, nt=nt, nh=nh, nkv=nkv)
    announce(f"attn seed={seed} ctx={ctx} nt={nt} nh={nh} nkv={nkv} kernel={kernel} chunk={chunk}")
    out = ops.attn_f16(dev_f32(q.reshape(nt, -1), dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev), pos0, nh, nkv,
                       kernel=kernel, chunk=chunk)
    got = host(out)
    want = oracle.attn(q.reshape(nt, -1), kb, vb, pos0, nh, nkv)
    return got, want


@pytest.mark.parametrize("seed,ctx,nt", [(0, 512, 1), (1, 8192, 1), (1, 8192, 4), (2, 4096 + 64, 64)])
def test_baseline_configs(dev, seed, ctx, nt):
    got, want = run_case(dev, seed, ctx, nt)
    err = np.abs(got - want).max()
    print(f"max_abs={err:.3g}")
    assert np.isfinite(got).all() and err <= TOL
    assert assert_argmax_agrees(got, want) == 0   # BASELINE config: no flip at all



@pytest.mark.parametrize("ctx,nt", [(128, 128), (64, 64), (256, 64), (4160, 64), (8192, 64), (1000, 40), (103, 3)])
def test_attn_q16_bit_equal(dev, ctx, nt):
    """it_attn_f16_q16 with q16 = f16(q * scale * log2 e) (the f32 product, RNE) equals it_attn_f16
    bit for bit: whole prompts and chunks in one pass, chunks with int16 key-split records, and a
    split-K call (nt < 16, q16 not read); and both stay at the oracle's bar."""
    nh, nkv, hd = 16, 2, 256
    pos0 = ctx - nt
    announce(f"attn q16 ctx={ctx} nt={nt}")
    q, kb, vb = attn_inputs(60 + ctx, ctx=ctx, nt=nt, nh=nh, nkv=nkv)
    q2 = np.ascontiguousarray(q.reshape(nt, -1), dtype=np.float32)
    s = np.float32(np.float32(1.0 / 16) * np.float32(1.4426950408889634))
    q16 = np.ascontiguousarray((q2.reshape(nt, nh, 2 * hd)[:, :, :hd] * s).astype(np.float16).reshape(nt, nh * hd))
    qd, kc, vc = dev_f32(q2, dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    a = host(ops.attn_f16(qd, kc, vc, pos0, nh, nkv))
    b = host(ops.attn_f16_q16(qd, torch.from_numpy(q16).to(dev), kc, vc, pos0, nh, nkv))
    np.testing.assert_array_equal(a, b)
    want = oracle.attn(q2, kb, vb, pos0, nh, nkv)
    assert np.abs(b - want).max() <= TOL

@pytest.mark.parametrize("ctx,nt,nh,nkv", [(1, 1, 16, 2), (65, 1, 16, 2), (100, 3, 16, 2), (64, 2, 24, 4),
                                           (300, 5, 8, 8), (129, 7, 4, 1), (777, 33, 16, 2), (64, 64, 16, 2)])
def test_ragged_and_group_shapes(dev, ctx, nt, nh, nkv):
    got, want = run_case(dev, 21, ctx, nt, nh, nkv, kernel=ops.KERNEL_SPLITK)
    assert np.abs(got - want).max() <= 1e-5


@pytest.mark.parametrize("nt", [1, 3, 4])
@pytest.mark.parametrize("chunk", [64, 128, 192, 256, 1024, 8192])
def test_split_invariance(dev, chunk, nt):
    """The result does not depend on how the keys are split (invariant of the LSE merge); chunks
    above 64 keys run several 64-key tiles per workgroup (online softmax across tiles)."""
    got, want = run_case(dev, 3, 2000, nt, kernel=ops.KERNEL_SPLITK, chunk=chunk)
    assert np.abs(got - want).max() <= 1e-5


@pytest.mark.parametrize("nh,nkv,hd", GEOMS)
@pytest.mark.parametrize("pos0,nt", CASES)
def test_r012_known_answer(dev, pos0, nt, nh, nkv, hd):
    """src/vk/r012_parity.rs:6-28 on the GPU path: RTZ KV append (bit-exact), then split-K attention
    against the f64 softmax oracle at the reference's own bound, max_abs < 2e-6."""
    announce(f"r012 pos0={pos0} nt={nt} nh={nh}")
    q, k, v = arena(pos0, nt, nh, nkv, hd)
    total = pos0 + nt
    kc = torch.zeros(total, nkv * hd, dtype=torch.int16, device=dev)
    vc = torch.zeros_like(kc)
    for start in range(0, total, 64):       # append in <= 64-row pieces like r012_parity.rs:12
        n = min(64, total - start)
        ops.kv_append_f16(dev_f32(k[start:start + n], dev), dev_f32(v[start:start + n], dev), kc, vc, start,
                          round_mode=1)
    kb = host(kc).view(np.uint16)
    np.testing.assert_array_equal(kb, f16_bits_rtz(k))
    np.testing.assert_array_equal(host(vc).view(np.uint16), f16_bits_rtz(v))
    got = host(ops.attn_f16(dev_f32(q, dev), kc, vc, pos0, nh, nkv, scale=1.0 / 16, kernel=ops.KERNEL_SPLITK))
    want = attn_f64(q, f16_to_f64(kb), f16_to_f64(host(vc).view(np.uint16)), pos0, nh, nkv, hd, 1.0 / 16)
    err = np.abs(got - want).max()
    print(f"r012 gpu max_abs={err:.3g}")
    assert np.isfinite(got).all() and err < 2e-6


@pytest.mark.parametrize("pos0,nt", [(0, 64), (0, 16), (63, 17), (4032, 64)])
@pytest.mark.parametrize("nh,nkv,hd", GEOMS)
def test_r012_flash(dev, pos0, nt, nh, nkv, hd):
    """The flash prefill kernel (f16 q and P on the matrix cores) on the r012 closed-form inputs,
    against the f64 softmax oracle at the north-star bound 2e-3."""
    announce(f"r012 flash pos0={pos0} nt={nt} nh={nh}")
    q, k, v = arena(pos0, nt, nh, nkv, hd)
    kb, vb = f16_bits_rtz(k), f16_bits_rtz(v)
    got = host(ops.attn_f16(dev_f32(q, dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev), pos0, nh, nkv,
                            scale=1.0 / 16, kernel=ops.KERNEL_FLASH))
    want = attn_f64(q, f16_to_f64(kb), f16_to_f64(vb), pos0, nh, nkv, hd, 1.0 / 16)
    err = np.abs(got - want).max()
    print(f"r012 flash max_abs={err:.3g}")
    assert np.isfinite(got).all() and err <= TOL


@pytest.mark.parametrize("ctx,nt,nh,nkv", [(16, 16, 16, 2), (100, 37, 16, 2), (300, 300, 16, 2), (333, 129, 24, 4),
                                           (200, 50, 8, 8), (1000, 64, 4, 1), (4096 + 64, 64, 16, 2)])
def test_flash_shapes(dev, ctx, nt, nh, nkv):
    got, want = run_case(dev, 31, ctx, nt, nh, nkv, kernel=ops.KERNEL_FLASH)
    err = np.abs(got - want).max()
    print(f"flash max_abs={err:.3g}")
    assert err <= TOL
    assert_argmax_agrees(got, want)


@pytest.mark.parametrize("chunk", [0, 64, 128, 192, 640, 4096, 8192])
def test_flash_key_splits(dev, chunk):
    """BASELINE config 3's first case (a 64-token chunk after 4096 cached positions, seed 2) through
    the flash kernel with its keys split (chunk 0 = the library's choice, 8192 = one pass): every
    split size gives the oracle's result within 2e-3 and the same downstream argmax."""
    got, want = run_case(dev, 2, 4096 + 64, 64, kernel=ops.KERNEL_FLASH, chunk=chunk)
    err = np.abs(got - want).max()
    print(f"flash split chunk={chunk} max_abs={err:.3g}")
    assert np.isfinite(got).all() and err <= TOL
    assert assert_argmax_agrees(got, want) == 0   # BASELINE config: no flip at all


def test_flash_whole_prompt_8192(dev):
    """BASELINE config 3 at full size (seed 2): one 8192-token causal call. The oracle checks the
    first and last 16 tokens; the whole output equals 128 chunked 64-token calls (split-K path)
    within the same tolerance (chunked prefill == single-pass causal)."""
    T = 8192
    q, kb, vb = attn_inputs(2, ctx=T, nt=T)
    announce("flash whole prompt 8192")
    qd = dev_f32(q.reshape(T, -1), dev)
    kc, vc = dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    whole = host(ops.attn_f16(qd, kc, vc, 0, 16, 2, kernel=ops.KERNEL_FLASH))
    for t0 in (0, T - 16):
        want = oracle.attn(q[t0:t0 + 16].reshape(16, -1), kb, vb, t0, 16, 2)
        assert np.abs(whole[t0:t0 + 16] - want).max() <= TOL
        assert assert_argmax_agrees(whole[t0:t0 + 16], want) == 0
    for kernel in (ops.KERNEL_SPLITK, ops.KERNEL_AUTO):   # split-K partials; flash (key splits past ~2k)
        chunked = np.concatenate([host(ops.attn_f16(qd[c:c + 64].contiguous(), kc, vc, c, 16, 2, kernel=kernel))
                                  for c in range(0, T, 64)])
        assert np.abs(whole - chunked).max() <= TOL


@pytest.mark.parametrize("chunk", [0, 64, 192, 640])
def test_flash_f32_records(dev, chunk):
    """The key-split flash path with lossless f32 records (kernel 3: the split-K kernels' 260-word
    {m, l, 0, 0, o[256]} form, merged by the f32 combine) at BASELINE config 3's first case: the
    oracle's result within 2e-3 with no argmax flip, the int16-record form with the same splits
    within its quantisation bound, and the same bits on a second call."""
    got, want = run_case(dev, 2, 4096 + 64, 64, kernel=ops.KERNEL_FLASH_F32, chunk=chunk)
    err = np.abs(got - want).max()
    print(f"flash f32 records chunk={chunk} max_abs={err:.3g}")
    assert np.isfinite(got).all() and err <= TOL
    assert assert_argmax_agrees(got, want) == 0
    q16, _ = run_case(dev, 2, 4096 + 64, 64, kernel=ops.KERNEL_FLASH, chunk=chunk)
    d = np.abs(q16 - got).max()
    print(f"int16 records vs f32 records: {d:.3g}")
    assert d <= 2e-4
    again, _ = run_case(dev, 2, 4096 + 64, 64, kernel=ops.KERNEL_FLASH_F32, chunk=chunk)
    np.testing.assert_array_equal(again, got)


def test_flash_int16_record_error_config3(dev):
    """BASELINE config 3 as configured (the 8192-token prompt as 128 chunks of 64 tokens, each given
    the reference arena's room): at every chunk position, the int16-record result against the same
    splits with f32 records (the quantisation error alone) and against the whole prompt in one pass.
    Prints the table per position; the int16 form stays within 2e-4 of the f32 records."""
    import ctypes
    from irontimber_amd._lib import call, lib
    T = 8192
    q, kb, vb = attn_inputs(2, ctx=T, nt=T)
    announce("flash int16 record error, 128 chunks of config 3")
    qd = dev_f32(q.reshape(T, -1), dev)
    kc, vc = dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    whole = host(ops.attn_f16(qd, kc, vc, 0, 16, 2, kernel=ops.KERNEL_FLASH))
    room = lib().it_attention_dispatch_room(T, 16, 64) * 4
    scr = torch.empty(room, dtype=torch.uint8, device=dev)
    rows, worst = [], 0.0
    for c in range(0, T, 64):
        k_, ch, nb = ctypes.c_int(), ctypes.c_int(), ctypes.c_size_t()
        assert lib().it_attn_plan(c, 64, 256, 16, 2, room, ctypes.byref(k_), ctypes.byref(ch), ctypes.byref(nb)) == 0
        qc = qd[c:c + 64].contiguous()
        out = torch.empty(64, 16 * 256, device=dev)
        call("it_attn_f16", qc.data_ptr(), 16 * 512, kc.data_ptr(), vc.data_ptr(), 512, c, 256, 16, 2, 64, 1.0 / 16,
             out.data_ptr(), 16 * 256, scr.data_ptr(), room, None)
        got = host(out)
        if ch.value:   # key splits: the same splits with f32 records
            ref = host(ops.attn_f16(qc, kc, vc, c, 16, 2, kernel=ops.KERNEL_FLASH_F32, chunk=ch.value))
            dq = float(np.abs(got - ref).max())
        else:
            dq = 0.0   # one pass: no records
        dw = float(np.abs(got - whole[c:c + 64]).max())
        rows.append((c, ch.value, dq, dw))
        worst = max(worst, dq)
        assert dw <= TOL
    print("pos0 chunk int16_vs_f32rec vs_one_pass")
    for r_ in rows:
        print(f"{r_[0]} {r_[1]} {r_[2]:.3g} {r_[3]:.3g}")
    print(f"max int16 quantisation error over the 128 chunks: {worst:.3g}")
    assert worst <= 2e-4


def test_decode_tokens_equal_single_pass(dev):
    """Token-by-token decode (nt = 1 at every position, split-K with the library's splits) equals
    one causal prefill pass over the same prompt (decode == single-pass causal)."""
    T = 160
    q, kb, vb = attn_inputs(5, ctx=T, nt=T)
    qd = dev_f32(q.reshape(T, -1), dev)
    kc, vc = dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    whole = host(ops.attn_f16(qd, kc, vc, 0, 16, 2, kernel=ops.KERNEL_FLASH))
    toks = np.concatenate([host(ops.attn_f16(qd[t:t + 1].contiguous(), kc, vc, t, 16, 2)) for t in range(T)])
    assert np.abs(whole - toks).max() <= TOL


def test_kv_append_rne_bits(dev):
    rng = np.random.default_rng(0)
    k = (rng.standard_normal((5, 512)) * 3).astype(np.float32)
    v = (rng.standard_normal((5, 512)) * 1e-3).astype(np.float32)
    kc = torch.full((9, 512), -1, dtype=torch.int16, device=dev)
    vc = torch.full((9, 512), -1, dtype=torch.int16, device=dev)
    ops.kv_append_f16(dev_f32(k, dev), dev_f32(v, dev), kc, vc, 3)
    kb, vb = host(kc).view(np.uint16), host(vc).view(np.uint16)
    np.testing.assert_array_equal(kb[3:8], f16_bits(k))
    np.testing.assert_array_equal(vb[3:8], f16_bits(v))
    assert (kb[:3] == 0xFFFF).all() and (kb[8:] == 0xFFFF).all()


def test_decode_sequence_matches_block(dev):
    """Token-by-token decode (nt=1 at pos0, pos0+1, ...) equals one nt-token call (MTP verify)."""
    ctx, nt = 1000, 4
    q, kb, vb = attn_inputs(5, ctx=ctx, nt=nt)
    qd = dev_f32(q.reshape(nt, -1), dev)
    kc, vc = dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    block = host(ops.attn_f16(qd, kc, vc, ctx - nt, 16, 2))
    for t in range(nt):
        one = host(ops.attn_f16(qd[t:t + 1].contiguous(), kc, vc, ctx - nt + t, 16, 2))
        np.testing.assert_allclose(one[0], block[t], atol=1e-6)


@pytest.mark.parametrize("ctx,nt", [(8192, 1), (8192, 4), (2048, 2)])
def test_two_phase_piece_layout_equals_single_call(dev, ctx, nt):
    """it_attn_partials_ex + it_attn_combine_ex with record layout 1 (the pieces it_attn_f16 uses
    for its wave merge) == it_attn_f16 bit for bit, and the records sit where the header says: the
    {m, l} pair of (t, h, s) equals the 260-word record's, piece (t, h, d/16, s) its o[d]."""
    from irontimber_amd._lib import call
    nh, nkv, chunk, pos0 = 16, 2, 64, ctx - nt
    announce(f"two-phase piece layout ctx={ctx} nt={nt}")
    q, kb, vb = attn_inputs(7, ctx=ctx, nt=nt)
    qd, kc, vc = dev_f32(q.reshape(nt, -1), dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    ref = host(ops.attn_f16(qd, kc, vc, pos0, nh, nkv, kernel=ops.KERNEL_SPLITK, chunk=chunk))
    nbytes = ops.attn_scratch_bytes(pos0, nt, nh, nkv, 256, ops.KERNEL_SPLITK, chunk)
    s = torch.cuda.current_stream().cuda_stream
    recs = []
    for layout in (0, 1):
        part = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
        out = torch.empty(nt, nh * 256, device=dev)
        call("it_attn_partials_ex", qd.data_ptr(), nh * 512, kc.data_ptr(), vc.data_ptr(), nkv * 256, pos0, 256, nh,
             nkv, nt, 1 / 16, part.data_ptr(), nbytes, chunk, layout, s)
        call("it_attn_combine_ex", qd.data_ptr(), nh * 512, part.data_ptr(), pos0, 256, nh, nt, chunk, layout,
             out.data_ptr(), nh * 256, s)
        np.testing.assert_array_equal(host(out), ref)
        recs.append(host(part))
    smax, rows = -(-ctx // chunk), nt * nh
    r0 = recs[0][:rows * smax * 260].reshape(rows, smax, 260)
    o1 = recs[1][:rows * smax * 256].reshape(rows, 16, smax, 16)
    h1 = recs[1][rows * smax * 256:rows * smax * 258].reshape(rows, smax, 2)
    for t in range(nt):   # splits token t sees (the others are never read)
        ns = (pos0 + t + chunk) // chunk
        th = slice(t * nh, (t + 1) * nh)
        np.testing.assert_array_equal(h1[th, :ns], r0[th, :ns, :2])
        np.testing.assert_array_equal(o1[th, :, :ns].transpose(0, 2, 1, 3).reshape(nh, ns, 256), r0[th, :ns, 4:])


def test_two_phase_abi_equals_single_call(dev):
    """it_attn_partials + it_attn_combine (the exchangeable split-K records) == it_attn_f16."""
    from irontimber_amd._lib import call
    ctx, nt, nh, nkv, chunk = 700, 3, 16, 2, 128
    q, kb, vb = attn_inputs(6, ctx=ctx, nt=nt)
    qd = dev_f32(q.reshape(nt, -1), dev)
    kc, vc = dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    ref = host(ops.attn_f16(qd, kc, vc, ctx - nt, nh, nkv, kernel=ops.KERNEL_SPLITK, chunk=chunk))
    nbytes = ops.attn_scratch_bytes(ctx - nt, nt, nh, nkv, 256, ops.KERNEL_SPLITK, chunk)
    part = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty(nt, nh * 256, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    call("it_attn_partials", qd.data_ptr(), nh * 512, kc.data_ptr(), vc.data_ptr(), nkv * 256, ctx - nt, 256, nh, nkv,
         nt, 1 / 16, part.data_ptr(), nbytes, chunk, s)
    call("it_attn_combine", qd.data_ptr(), nh * 512, part.data_ptr(), ctx - nt, 256, nh, nt, chunk, out.data_ptr(),
         nh * 256, s)
    np.testing.assert_array_equal(host(out), ref)


def _two_phase_f32(dev, qd, kc, vc, pos0, nt, nh, nkv, chunk):
    """it_attn_partials + it_attn_combine: the split-K path with the 260-word f32 records."""
    from irontimber_amd._lib import call
    nbytes = ops.attn_scratch_bytes(pos0, nt, nh, nkv, 256, ops.KERNEL_SPLITK, chunk)
    part = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    out = torch.empty(nt, nh * 256, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    call("it_attn_partials", qd.data_ptr(), nh * 512, kc.data_ptr(), vc.data_ptr(), nkv * 256, pos0, 256, nh, nkv,
         nt, 1 / 16, part.data_ptr(), nbytes, chunk, s)
    call("it_attn_combine", qd.data_ptr(), nh * 512, part.data_ptr(), pos0, 256, nh, nt, chunk, out.data_ptr(),
         nh * 256, s)
    return host(out)


@pytest.mark.parametrize("ctx,nt", [(1100, 1), (4096, 2), (8192, 1), (8192, 4), (16384, 1)])
def test_piece_records_equal_f32_records(dev, ctx, nt):
    """Decode and verify calls of it_attn_f16 whose merge is the wave merge (9-256 splits, at most
    256 rows) lay their split records out in 64-byte pieces per (row, 16-dim block, split): the
    same f32 values merged in the same order, so the output equals it_attn_partials +
    it_attn_combine (the 260-word records) bit for bit, at the oracle's bar."""
    nh, nkv, pos0 = 16, 2, ctx - nt
    announce(f"piece records ctx={ctx} nt={nt}")
    q, kb, vb = attn_inputs(70 + ctx + nt, ctx=ctx, nt=nt, nh=nh, nkv=nkv)
    qd, kc, vc = dev_f32(q.reshape(nt, -1), dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev)
    got = host(ops.attn_f16(qd, kc, vc, pos0, nh, nkv, kernel=ops.KERNEL_SPLITK, chunk=64))
    np.testing.assert_array_equal(got, _two_phase_f32(dev, qd, kc, vc, pos0, nt, nh, nkv, 64))
    want = oracle.attn(q.reshape(nt, -1), kb, vb, pos0, nh, nkv)
    assert np.isfinite(got).all() and np.abs(got - want).max() <= TOL
    assert assert_argmax_agrees(got, want) == 0


@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_piece_records_nonfinite(dev, bad):
    """A NaN or infinite V value at ctx 8192 (piece-layout records, wave merge): every row that sees
    the key gets a non-finite output in that dim, the other KV head stays finite."""
    nh, nkv, nt, ctx = 16, 2, 1, 8192
    announce(f"piece records nonfinite bad={bad}")
    q, kb, vb = attn_inputs(9, ctx=ctx, nt=nt, nh=nh, nkv=nkv)
    vb = vb.copy()
    vb[5000, 3] = np.float16(bad).view(np.uint16)   # dim 3 of KV head 0
    got = host(ops.attn_f16(dev_f32(q.reshape(nt, -1), dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev), ctx - nt,
                            nh, nkv)).reshape(nh, 256)
    assert not np.isfinite(got[:nh // nkv, 3]).any()
    assert np.isfinite(got[nh // nkv:]).all()


@pytest.mark.parametrize("pos0,nt,cap", [(3968, 64, 8192), (4032, 64, 8192), (8128, 64, 8192), (3977, 64, 4041),
                                         (245, 13, 258), (8188, 4, 8192), (4096, 64, 0), (7680, 512, 8192),
                                         (7000, 300, 7300)])
def test_reference_room_is_enough(dev, pos0, nt, cap):
    """it_attn_f16 with scratch of exactly the reference arena's room (attention_dispatch_room at
    capacity `cap`, src/vk/mod.rs:148-150, 714-716; cap 0 = no scratch at all): the split grows until
    the records fit, nothing past the room is written, and the result matches the oracle."""
    from irontimber_amd import _lib
    lib = _lib.lib()
    ctx = pos0 + nt
    room = lib.it_attention_dispatch_room(cap, 16, nt) * 4 if cap else 0
    announce(f"attn room pos0={pos0} nt={nt} cap={cap} room={room} preferred={ops.attn_scratch_bytes(pos0, nt, 16, 2)}")
    q, kb, vb = attn_inputs(2, ctx=ctx, nt=nt)
    guard = 1 << 16
    buf = torch.full((room + guard,), 0x5A, dtype=torch.uint8, device=dev)
    scratch = buf if room else None
    qd = dev_f32(q.reshape(nt, -1), dev)
    out = torch.empty(nt, 16 * 256, device=dev)
    kc, vc = dev_f16bits(kb, dev), dev_f16bits(vb, dev)   # held: a freed block could be reused by the next upload
    _lib.call("it_attn_f16", qd.data_ptr(), 16 * 512, kc.data_ptr(), vc.data_ptr(),
              512, pos0, 256, 16, 2, nt, 1.0 / 16, out.data_ptr(), 16 * 256,
              scratch.data_ptr() if scratch is not None else None, room, None)
    got = host(out)
    assert bool((buf[room:] == 0x5A).all()), "scratch written past the room"
    want = oracle.attn(q.reshape(nt, -1), kb, vb, pos0, 16, 2)
    err = np.abs(got - want).max()
    print(f"max_abs={err:.3g}")
    assert np.isfinite(got).all() and err <= TOL
    assert assert_argmax_agrees(got, want) == 0


@pytest.mark.parametrize("kernel,chunk", [(ops.KERNEL_SPLITK, 0), (ops.KERNEL_FLASH, 0), (ops.KERNEL_FLASH, 64),
                                          (ops.KERNEL_FLASH, 8192)])
@pytest.mark.parametrize("bad", [float("nan"), float("inf")])
def test_nonfinite_value_row_propagates(dev, kernel, chunk, bad):
    """A NaN or infinite value in V (one key's row of one KV head) reaches every output row that
    sees that key, as in the reference's arithmetic (cpu.rs:266-270 sums e_p v_p): no path may
    quantise it away (the flash key-split records hold O as int16 against the row's max |O|, and
    that maximum is taken so that NaN and infinity survive it). Rows of tokens whose visible keys
    end before the key's 64-key tile, and the other KV head's rows, stay finite. (Rows that share
    the key's tile but not the key may turn NaN too: their P is 0 there and the matrix product
    computes 0 * NaN; cpu.rs never touches keys a row cannot see.)"""
    nh, nkv, nt, pos0 = 16, 2, 64, 1000
    ctx = pos0 + nt
    announce(f"nonfinite V kernel={kernel} chunk={chunk} bad={bad}")
    q, kb, vb = attn_inputs(5, ctx=ctx, nt=nt, nh=nh, nkv=nkv)
    key = pos0 + 40                       # seen by tokens 40.. of the chunk; its tile starts at 1024
    vb = vb.copy()
    vb[key, 3] = np.float16(bad).view(np.uint16)   # dim 3 of KV head 0
    got = host(ops.attn_f16(dev_f32(q.reshape(nt, -1), dev), dev_f16bits(kb, dev), dev_f16bits(vb, dev), pos0, nh,
                            nkv, kernel=kernel, chunk=chunk))
    g = got.reshape(nt, nh, 256)
    head0 = slice(0, nh // nkv)
    assert not np.isfinite(g[40:, head0, 3]).any()          # every row that sees the key
    assert np.isfinite(g[:1024 - pos0]).all()                 # tokens whose keys end before its tile
    assert np.isfinite(g[:, nh // nkv:]).all()                # the other KV head
