"""Torch-tensor front end over the C ABI (device memory and streams come from PyTorch-ROCm).

Each function validates dtypes/devices/contiguity, then calls the matching `it_*` entry point on
torch's current stream. Buffer layouts and semantics are those of include/it_attn.h.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import call, lib

KERNEL_AUTO, KERNEL_SPLITK, KERNEL_FLASH, KERNEL_FLASH_F32 = 0, 1, 2, 3


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, dtype: torch.dtype, name: str):
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def kv_append_f16(k: torch.Tensor, v: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int,
                  round_mode: int = 0) -> None:
    """Append k, v [nt, kvd] f32 to the f16 caches kc, vc [ctx, kvd] (stored as int16 bits or f16)."""
    _need(k, torch.float32, "k"); _need(v, torch.float32, "v")
    nt, kvd = k.shape
    for c in (kc, vc):
        if c.dtype not in (torch.float16, torch.int16) or not c.is_contiguous() or c.shape[-1] != kvd:
            raise ValueError("kc/vc must be contiguous [ctx, kvd] f16")
        if c.shape[0] < pos0 + nt:
            raise ValueError("cache too short")
    call("it_kv_append_f16", k.data_ptr(), v.data_ptr(), kvd, kc.data_ptr(), vc.data_ptr(), pos0, nt, kvd,
         round_mode, _stream())


def attn_prep_f16(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int,
                  nh: int, nkv: int, q_norm: torch.Tensor | None = None, k_norm: torch.Tensor | None = None,
                  eps: float = 1e-6, n_rot: int = 64, theta_scale: float | None = None, rope_base: float = 1e7,
                  sections=(11, 11, 10, 0), round_mode: int = 0) -> None:
    """Norm + rope of q (in place, q [nt, nh*2*hd]) and k [nt, nkv*hd], then the f16 append of k and
    v to kc/vc at rows pos0.. (it_attn_prep_f16). theta_scale defaults to rope_base^(-2/n_rot) in f32."""
    _need(q, torch.float32, "q"); _need(k, torch.float32, "k"); _need(v, torch.float32, "v")
    nt, kvd = k.shape
    hd = kvd // nkv
    if q.shape != (nt, nh * 2 * hd) or v.shape != k.shape:
        raise ValueError("q must be [nt, nh*2*hd] and v the shape of k [nt, nkv*hd]")
    for c in (kc, vc):
        if c.dtype not in (torch.float16, torch.int16) or not c.is_contiguous() or c.shape[-1] != kvd:
            raise ValueError("kc/vc must be contiguous [ctx, kvd] f16")
        if c.shape[0] < pos0 + nt:
            raise ValueError("cache too short")
    for w, n in ((q_norm, "q_norm"), (k_norm, "k_norm")):
        if w is not None:
            _need(w, torch.float32, n)
            if w.numel() != hd:
                raise ValueError(f"{n} must hold head_dim floats")
    if theta_scale is None:
        from .synth import rope_theta_scale
        theta_scale = rope_theta_scale(rope_base, n_rot)
    s = list(sections) + [0] * (4 - len(sections))
    call("it_attn_prep_f16", q.data_ptr(), q.shape[1], k.data_ptr(), v.data_ptr(), kvd, _ptr(q_norm), _ptr(k_norm),
         float(eps), kc.data_ptr(), vc.data_ptr(), kvd, pos0, hd, nh, nkv, nt, n_rot, float(theta_scale), *s[:4],
         round_mode, _stream())


def attn_prep_f16_q16(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int,
                      nh: int, nkv: int, scale: float | None = None, q_norm: torch.Tensor | None = None,
                      k_norm: torch.Tensor | None = None, eps: float = 1e-6, n_rot: int = 64,
                      theta_scale: float | None = None, rope_base: float = 1e7, sections=(11, 11, 10, 0),
                      round_mode: int = 0) -> torch.Tensor:
    """attn_prep_f16 that also returns q16 [nt, nh*hd] f16 = f16(q' * scale * log2(e)), the flash
    prefill kernel's query operand for attn_f16_q16 with the same scale (it_attn_prep_f16_q16)."""
    _need(q, torch.float32, "q"); _need(k, torch.float32, "k"); _need(v, torch.float32, "v")
    nt, kvd = k.shape
    hd = kvd // nkv
    if q.shape != (nt, nh * 2 * hd) or v.shape != k.shape:
        raise ValueError("q must be [nt, nh*2*hd] and v the shape of k [nt, nkv*hd]")
    for c in (kc, vc):
        if c.dtype not in (torch.float16, torch.int16) or not c.is_contiguous() or c.shape[-1] != kvd:
            raise ValueError("kc/vc must be contiguous [ctx, kvd] f16")
        if c.shape[0] < pos0 + nt:
            raise ValueError("cache too short")
    if scale is None:
        scale = 1.0 / hd ** 0.5
    if theta_scale is None:
        from .synth import rope_theta_scale
        theta_scale = rope_theta_scale(rope_base, n_rot)
    q16 = torch.empty(nt, nh * hd, device=q.device, dtype=torch.float16)
    s = list(sections) + [0] * (4 - len(sections))
    call("it_attn_prep_f16_q16", q.data_ptr(), q.shape[1], k.data_ptr(), v.data_ptr(), kvd, _ptr(q_norm),
         _ptr(k_norm), float(eps), kc.data_ptr(), vc.data_ptr(), kvd, pos0, hd, nh, nkv, nt, n_rot, float(theta_scale),
         *s[:4], round_mode, q16.data_ptr(), nh * hd, float(scale), _stream())
    return q16


def attn_prep_f32kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int,
                    row0: int, nh: int, nkv: int, q_norm: torch.Tensor | None = None,
                    k_norm: torch.Tensor | None = None, eps: float = 1e-6, n_rot: int = 64,
                    theta_scale: float | None = None, rope_base: float = 1e7, sections=(11, 11, 10, 0)) -> None:
    """attn_prep_f16 for an f32 cache: rope at positions pos0.., K/V rows stored at cache rows row0..
    (the MTP head stores position p in row p - 1)."""
    _need(q, torch.float32, "q"); _need(k, torch.float32, "k"); _need(v, torch.float32, "v")
    _need(kc, torch.float32, "kc"); _need(vc, torch.float32, "vc")
    nt, kvd = k.shape
    hd = kvd // nkv
    if q.shape != (nt, nh * 2 * hd) or v.shape != k.shape:
        raise ValueError("q must be [nt, nh*2*hd] and v the shape of k [nt, nkv*hd]")
    for c in (kc, vc):
        if c.shape[-1] != kvd or c.shape[0] < row0 + nt:
            raise ValueError("kc/vc must be [rows >= row0 + nt, kvd] f32")
    if theta_scale is None:
        from .synth import rope_theta_scale
        theta_scale = rope_theta_scale(rope_base, n_rot)
    s = list(sections) + [0] * (4 - len(sections))
    call("it_attn_prep_f32kv", q.data_ptr(), q.shape[1], k.data_ptr(), v.data_ptr(), kvd, _ptr(q_norm), _ptr(k_norm),
         float(eps), kc.data_ptr(), vc.data_ptr(), kvd, pos0, row0, hd, nh, nkv, nt, n_rot, float(theta_scale), *s[:4],
         _stream())


def attn_f32kv(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int, nh: int, nkv: int,
               scale: float | None = None, out: torch.Tensor | None = None,
               scratch: torch.Tensor | None = None) -> torch.Tensor:
    """q [nt, nh*2*hd] f32 (q | gate per head), kc/vc [rows, nkv*hd] f32 -> out [nt, nh*hd] f32;
    query t sees rows 0..pos0+t."""
    _need(q, torch.float32, "q"); _need(kc, torch.float32, "kc"); _need(vc, torch.float32, "vc")
    nt = q.shape[0]
    hd = q.shape[-1] // (2 * nh)
    kvd = nkv * hd
    for c in (kc, vc):
        if c.shape[-1] != kvd or c.shape[0] < pos0 + nt:
            raise ValueError("kc/vc must be [rows >= pos0 + nt, nkv*hd] f32")
    if scale is None:
        scale = 1.0 / hd ** 0.5
    if out is None:
        out = torch.empty(nt, nh * hd, device=q.device, dtype=torch.float32)
    if scratch is None:
        need = lib().it_attn_f32kv_scratch_bytes(pos0, nt, hd, nh, nkv)
        scratch = torch.empty(max(need, 16), device=q.device, dtype=torch.uint8)
    sp, sb = (scratch.data_ptr(), scratch.numel() * scratch.element_size()) if scratch.numel() else (None, 0)
    call("it_attn_f32kv", q.data_ptr(), nh * 2 * hd, kc.data_ptr(), vc.data_ptr(), kvd, pos0, hd, nh, nkv, nt,
         float(scale), out.data_ptr(), nh * hd, sp, sb, _stream())
    return out


def attn_scratch_bytes(pos0: int, nt: int, nh: int, nkv: int, hd: int = 256, kernel: int = KERNEL_AUTO,
                       chunk: int = 0) -> int:
    return lib().it_attn_scratch_bytes_ex(pos0, nt, hd, nh, nkv, kernel, chunk)


def attn_f16(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int, nh: int, nkv: int,
             scale: float | None = None, out: torch.Tensor | None = None, scratch: torch.Tensor | None = None,
             kernel: int = KERNEL_AUTO, chunk: int = 0) -> torch.Tensor:
    """q [nt, nh*2*hd] f32 (q | gate per head), kc/vc [ctx, nkv*hd] f16 -> out [nt, nh*hd] f32."""
    _need(q, torch.float32, "q")
    nt = q.shape[0]
    hd = q.shape[-1] // (2 * nh) if q.dim() == 2 else q.shape[-1] // 2
    kvd = nkv * hd
    if scale is None:
        scale = 1.0 / hd ** 0.5
    for c in (kc, vc):
        if c.dtype not in (torch.float16, torch.int16) or not c.is_contiguous() or c.shape[-1] != kvd:
            raise ValueError("kc/vc must be contiguous [ctx, nkv*hd] f16")
        if c.shape[0] < pos0 + nt:
            raise ValueError("cache shorter than pos0 + nt")
    if out is None:
        out = torch.empty(nt, nh * hd, device=q.device, dtype=torch.float32)
    _need(out, torch.float32, "out")
    need = attn_scratch_bytes(pos0, nt, nh, nkv, hd, kernel, chunk)
    if scratch is None and need:
        scratch = torch.empty(need, device=q.device, dtype=torch.uint8)
    nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    call("it_attn_f16_ex", q.data_ptr(), nh * 2 * hd, kc.data_ptr(), vc.data_ptr(), kvd, pos0, hd, nh, nkv, nt,
         float(scale), out.data_ptr(), nh * hd, _ptr(scratch), nbytes, kernel, chunk, _stream())
    return out


def attn_f16_q16(q: torch.Tensor, q16: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int, nh: int, nkv: int,
                 scale: float | None = None, out: torch.Tensor | None = None,
                 scratch: torch.Tensor | None = None) -> torch.Tensor:
    """attn_f16 with the flash kernel's query operand given as q16 [nt, nh*hd] f16 (attn_prep_f16_q16
    with the same scale, or f16(q * scale * log2(e))); q still gives the gates (it_attn_f16_q16)."""
    _need(q, torch.float32, "q")
    nt = q.shape[0]
    hd = q.shape[-1] // (2 * nh)
    kvd = nkv * hd
    if scale is None:
        scale = 1.0 / hd ** 0.5
    if q16.dtype != torch.float16 or not q16.is_contiguous() or q16.shape != (nt, nh * hd):
        raise ValueError("q16 must be contiguous [nt, nh*hd] f16")
    for c in (kc, vc):
        if c.dtype not in (torch.float16, torch.int16) or not c.is_contiguous() or c.shape[-1] != kvd:
            raise ValueError("kc/vc must be contiguous [ctx, nkv*hd] f16")
        if c.shape[0] < pos0 + nt:
            raise ValueError("cache shorter than pos0 + nt")
    if out is None:
        out = torch.empty(nt, nh * hd, device=q.device, dtype=torch.float32)
    _need(out, torch.float32, "out")
    if scratch is None:
        need = attn_scratch_bytes(pos0, nt, nh, nkv, hd)
        scratch = torch.empty(need, device=q.device, dtype=torch.uint8) if need else None
    nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    call("it_attn_f16_q16", q.data_ptr(), nh * 2 * hd, q16.data_ptr(), nh * hd, kc.data_ptr(), vc.data_ptr(), kvd,
         pos0, hd, nh, nkv, nt, float(scale), out.data_ptr(), nh * hd, _ptr(scratch), nbytes, _stream())
    return out


def attn_mailbox(ctx: int, nt: int, nh: int, device) -> torch.Tensor:
    """A mailbox for attn_f16_mailbox (decode / verify rows up to nt at context up to ctx, nh
    heads), initialised on the current stream. Keep one per stream of calls."""
    nbytes = lib().it_attn_mailbox_bytes(ctx, nt, nh)
    mb = torch.empty(nbytes, device=device, dtype=torch.uint8)
    call("it_attn_mailbox_init", mb.data_ptr(), nbytes, _stream())
    return mb


def attn_mailbox_poisoned(mb: torch.Tensor) -> bool:
    """True if a one-launch merge in this mailbox ever gave up waiting (synchronises the stream)."""
    flag = ctypes.c_int(0)
    call("it_attn_mailbox_poisoned", mb.data_ptr(), ctypes.addressof(flag), _stream())
    return bool(flag.value)


def attn_mailbox_would_launch(pos0: int, nt: int, nh: int, nkv: int, mailbox: torch.Tensor, hd: int = 256) -> bool:
    """Whether attn_f16_mailbox takes the one-launch form for this geometry and mailbox."""
    return bool(lib().it_attn_mailbox_would_launch(pos0, nt, hd, nh, nkv, mailbox.numel()))


def attn_f16_mailbox(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos0: int, nh: int, nkv: int,
                     mailbox: torch.Tensor, scale: float | None = None, out: torch.Tensor | None = None,
                     scratch: torch.Tensor | None = None) -> torch.Tensor:
    """attn_f16 with decode in one launch through `mailbox` (attn_mailbox) where the
    geometry allows it; otherwise the same as attn_f16 with `scratch`."""
    _need(q, torch.float32, "q")
    nt = q.shape[0]
    hd = q.shape[-1] // (2 * nh)
    kvd = nkv * hd
    if scale is None:
        scale = 1.0 / hd ** 0.5
    for c in (kc, vc):
        if c.dtype not in (torch.float16, torch.int16) or not c.is_contiguous() or c.shape[-1] != kvd:
            raise ValueError("kc/vc must be contiguous [ctx, nkv*hd] f16")
        if c.shape[0] < pos0 + nt:
            raise ValueError("cache shorter than pos0 + nt")
    if out is None:
        out = torch.empty(nt, nh * hd, device=q.device, dtype=torch.float32)
    _need(out, torch.float32, "out")
    if scratch is None:
        need = attn_scratch_bytes(pos0, nt, nh, nkv, hd)
        scratch = torch.empty(max(need, 1), device=q.device, dtype=torch.uint8)
    call("it_attn_f16_mailbox", q.data_ptr(), nh * 2 * hd, kc.data_ptr(), vc.data_ptr(), kvd, pos0, hd, nh, nkv, nt,
         float(scale), out.data_ptr(), nh * hd, mailbox.data_ptr(), mailbox.numel(), scratch.data_ptr(),
         scratch.numel(), _stream())
    return out


def _ckpt(ckpt, like: torch.Tensor):
    if ckpt is not None:
        _need(ckpt, torch.float32, "ckpt")
        if ckpt.numel() != like.numel():
            raise ValueError("ckpt must have the shape of the state it snapshots")


def gdn_conv(x: torch.Tensor, w: torch.Tensor, state: torch.Tensor, out: torch.Tensor | None = None,
             ckpt: torch.Tensor | None = None, ckpt_after: int = 0) -> torch.Tensor:
    """x [nt, cd] f32, w [cd, K], state [K-1, cd] (updated in place) -> silu(conv) [nt, cd].
    ckpt (optional, shape of state) receives the state after token ckpt_after."""
    _need(x, torch.float32, "x"); _need(w, torch.float32, "w"); _need(state, torch.float32, "state")
    _ckpt(ckpt, state)
    nt, cd = x.shape
    K = w.shape[1]
    if out is None:
        out = torch.empty_like(x)
    if ckpt is None:
        call("it_gdn_conv", x.data_ptr(), cd, w.data_ptr(), state.data_ptr(), out.data_ptr(), cd, cd, nt, K, _stream())
    else:
        call("it_gdn_conv_ckpt", x.data_ptr(), cd, w.data_ptr(), state.data_ptr(), out.data_ptr(), cd, cd, nt, K,
             ckpt.data_ptr(), ckpt_after, _stream())
    return out


def gdn_conv_l2norm(x: torch.Tensor, w: torch.Tensor, state: torch.Tensor, nnorm: int, eps: float = 1e-6,
                    out: torch.Tensor | None = None, ckpt: torch.Tensor | None = None,
                    ckpt_after: int = 0) -> torch.Tensor:
    """gdn_conv then l2norm_heads(out, nnorm, 128, eps) in one pass (x [nt, cd], cd % 128 == 0);
    ckpt as for gdn_conv."""
    _need(x, torch.float32, "x"); _need(w, torch.float32, "w"); _need(state, torch.float32, "state")
    _ckpt(ckpt, state)
    nt, cd = x.shape
    K = w.shape[1]
    if out is None:
        out = torch.empty_like(x)
    if ckpt is None:
        call("it_gdn_conv_l2norm", x.data_ptr(), cd, w.data_ptr(), state.data_ptr(), out.data_ptr(), cd, cd, nt, K,
             nnorm, float(eps), _stream())
    else:
        call("it_gdn_conv_l2norm_ckpt", x.data_ptr(), cd, w.data_ptr(), state.data_ptr(), out.data_ptr(), cd, cd, nt,
             K, nnorm, float(eps), ckpt.data_ptr(), ckpt_after, _stream())
    return out


def l2norm_heads(x: torch.Tensor, nheads: int, d: int, eps: float = 1e-6) -> torch.Tensor:
    """In place on the first nheads*d columns of each row of x [nt, C]."""
    _need(x, torch.float32, "x")
    call("it_l2norm_heads", x.data_ptr(), x.shape[1], nheads, d, x.shape[0], float(eps), _stream())
    return x


def gdn_decode_fused(x, w, conv_state_in, conv_state_out, beta_raw, alpha_raw, dt, a, state, nv: int, nk: int,
                     eps: float = 1e-6, out=None, ckpt_state=None, ckpt_conv=None, ckpt_after: int = 0):
    """One launch for a GDN decode layer (1 <= nt <= 4 tokens): gdn_conv_l2norm(x, w, ...) then
    gdn_step, with the conv state read from conv_state_in and the new one written to
    conv_state_out (a different buffer). x [nt, (2nk+nv)*128], state updated in place -> out
    [nt, nv*128]. ckpt_state / ckpt_conv (optional, together): both states after token ckpt_after
    (the MTP verify checkpoint)."""
    for t, n in ((x, "x"), (w, "w"), (conv_state_in, "conv_state_in"), (conv_state_out, "conv_state_out"),
                 (beta_raw, "beta_raw"), (alpha_raw, "alpha_raw"), (dt, "dt"), (a, "a"), (state, "state")):
        _need(t, torch.float32, n)
    nt, cd = x.shape
    S = state.shape[-1]
    if out is None:
        out = torch.empty(nt, nv * S, device=x.device, dtype=torch.float32)
    args = [x.data_ptr(), cd, w.data_ptr(), w.shape[1], conv_state_in.data_ptr(), conv_state_out.data_ptr(),
            beta_raw.data_ptr(), alpha_raw.data_ptr(), beta_raw.shape[1], dt.data_ptr(), a.data_ptr(), state.data_ptr(),
            out.data_ptr(), out.shape[1], nt, nv, nk, S, float(eps)]
    if ckpt_state is None and ckpt_conv is None:
        call("it_gdn_decode_fused", *args, _stream())
    else:
        _ckpt(ckpt_state, state)
        _ckpt(ckpt_conv, conv_state_in)
        call("it_gdn_decode_fused_ckpt", *args, ckpt_state.data_ptr(), ckpt_conv.data_ptr(), ckpt_after, _stream())
    return out


def gdn_step(co, beta_raw, alpha_raw, dt, a, state, nv: int, nk: int, out=None, chunked: bool = False,
             scratch=None, ckpt=None, ckpt_after: int = 0):
    """co [nt, (2nk+nv)S], beta_raw/alpha_raw [nt, nv], dt/a [nv], state [nv, S, S] (in place)
    -> out [nt, nv*S]. chunked=True uses the chunk-64 scan (it_gdn_chunked). ckpt (optional, shape
    of state; token-sequential kernel only) receives the state after token ckpt_after."""
    _ckpt(ckpt, state)
    if ckpt is not None and chunked:
        raise ValueError("the checkpoint is a feature of the token-sequential kernel")
    for t, n in ((co, "co"), (beta_raw, "beta_raw"), (alpha_raw, "alpha_raw"), (dt, "dt"), (a, "a"), (state, "state")):
        _need(t, torch.float32, n)
    nt = co.shape[0]
    S = state.shape[-1]
    if out is None:
        out = torch.empty(nt, nv * S, device=co.device, dtype=torch.float32)
    args = [co.data_ptr(), co.shape[1], beta_raw.data_ptr(), alpha_raw.data_ptr(), beta_raw.shape[1], dt.data_ptr(),
            a.data_ptr(), state.data_ptr(), out.data_ptr(), out.shape[1], nt, nv, nk, S]
    if chunked:
        need = lib().it_gdn_chunked_scratch_bytes(nt, nv, S)
        if scratch is None and need:
            scratch = torch.empty(need, device=co.device, dtype=torch.uint8)
        nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
        call("it_gdn_chunked", *args, _ptr(scratch), nbytes, _stream())
    elif ckpt is not None:
        call("it_gdn_step_ckpt", *args, ckpt.data_ptr(), ckpt_after, _stream())
    else:
        call("it_gdn_step", *args, _stream())
    return out


def gdn_prefill(x, w, conv_state, beta_raw, alpha_raw, dt, a, state, nv: int, nk: int, eps: float = 1e-6, out=None,
                scratch=None):
    """The GDN layer over a prompt chunk in one call (it_gdn_prefill): conv + SiLU + q/k L2 kept as
    f16 in scratch, then the chunk-64 scan. x [nt, cd] f32, w [cd, K], conv_state [K-1, cd] and
    state [nv, S, S] updated in place -> out [nt, nv*S]."""
    for t, n in ((x, "x"), (w, "w"), (conv_state, "conv_state"), (beta_raw, "beta_raw"), (alpha_raw, "alpha_raw"),
                 (dt, "dt"), (a, "a"), (state, "state")):
        _need(t, torch.float32, n)
    nt = x.shape[0]
    S = state.shape[-1]
    if out is None:
        out = torch.empty(nt, nv * S, device=x.device, dtype=torch.float32)
    need = lib().it_gdn_prefill_scratch_bytes(nt, nv, nk, S)
    if scratch is None and need:
        scratch = torch.empty(need, device=x.device, dtype=torch.uint8)
    nbytes = 0 if scratch is None else scratch.numel() * scratch.element_size()
    call("it_gdn_prefill", x.data_ptr(), x.shape[1], w.data_ptr(), w.shape[1], conv_state.data_ptr(),
         beta_raw.data_ptr(), alpha_raw.data_ptr(), beta_raw.shape[1], dt.data_ptr(), a.data_ptr(), state.data_ptr(),
         out.data_ptr(), out.shape[1], nt, nv, nk, S, float(eps), _ptr(scratch), nbytes, _stream())
    return out


def gdn_gated_rmsnorm(o: torch.Tensor, z: torch.Tensor, w: torch.Tensor, nv: int, eps: float = 1e-6,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """o, z [nt, nv*128], w [128] -> o / rms(o) * w * silu(z) per 128-wide head row (out may be o)."""
    _need(o, torch.float32, "o"); _need(z, torch.float32, "z"); _need(w, torch.float32, "w")
    if out is None:
        out = torch.empty_like(o)
    call("it_gdn_gated_rmsnorm", o.data_ptr(), o.shape[1], z.data_ptr(), z.shape[1], w.data_ptr(), float(eps),
         out.data_ptr(), out.shape[1], nv, 128, o.shape[0], _stream())
    return out


def gdn_step_gated(co, beta_raw, alpha_raw, dt, a, state, nv: int, nk: int, z=None, norm_w=None, eps: float = 1e-6,
                   out=None, ckpt=None, ckpt_after: int = 0):
    """The recurrence with one workgroup per V head and, when z is given, the gated RMSNorm
    (o / rms(o) * norm_w * silu(z)) fused into the output write (it_gdn_step_gated)."""
    for t, n in ((co, "co"), (beta_raw, "beta_raw"), (alpha_raw, "alpha_raw"), (dt, "dt"), (a, "a"), (state, "state")):
        _need(t, torch.float32, n)
    if z is not None:
        _need(z, torch.float32, "z"); _need(norm_w, torch.float32, "norm_w")
    _ckpt(ckpt, state)
    nt = co.shape[0]
    S = state.shape[-1]
    if out is None:
        out = torch.empty(nt, nv * S, device=co.device, dtype=torch.float32)
    call("it_gdn_step_gated", co.data_ptr(), co.shape[1], beta_raw.data_ptr(), alpha_raw.data_ptr(), beta_raw.shape[1],
         dt.data_ptr(), a.data_ptr(), state.data_ptr(), out.data_ptr(), out.shape[1], nt, nv, nk, S, _ptr(z),
         0 if z is None else z.shape[1], _ptr(norm_w), float(eps), _ptr(ckpt), ckpt_after, _stream())
    return out


def gdn_rollback(ck_conv: torch.Tensor | None, conv_state: torch.Tensor | None, ck_ssm: torch.Tensor | None,
                 ssm: torch.Tensor | None) -> None:
    """Restore the checkpointed conv and SSM states after a rejected draft (it_gdn_rollback)."""
    cw = 0 if conv_state is None else conv_state.numel()
    sw = 0 if ssm is None else ssm.numel()
    for c, t in ((ck_conv, conv_state), (ck_ssm, ssm)):
        if t is not None and (c is None or c.numel() != t.numel()):
            raise ValueError("checkpoint and state sizes differ")
    call("it_gdn_rollback", _ptr(ck_conv), _ptr(conv_state), cw, _ptr(ck_ssm), _ptr(ssm), sw, _stream())
