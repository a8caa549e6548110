"""CPU tests of the C-ABI boundary (no GPU, no kernel launches).

libsphkv.so must load, export every function include/sphkv.h declares, and the
ctypes table must agree with the header on argument counts.  The argument
checks run on the host before any HIP call, so their error behaviour is tested
here: a bad call returns a negative status and leaves a message.
"""
import ctypes
import os
import re

import pytest

import sphkv_lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "sphkv.h")


def header_functions():
    """name -> number of parameters of every function declared in sphkv.h."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(sphkv_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        name, params = m.group(1), m.group(2).strip()
        out[name] = 0 if params in ("", "void") else len(params.split(","))
    return out


def test_header_parses():
    fns = header_functions()
    assert "sphkv_decode_paged" in fns and "sphkv_encode_pages" in fns
    assert len(fns) >= 8


def test_library_exports_every_declared_symbol():
    lib = sphkv_lib.load()
    for name in header_functions():
        assert hasattr(lib, name), f"{name} declared in sphkv.h but not exported"


def test_ctypes_table_matches_header():
    fns = header_functions()
    assert set(sphkv_lib.SIGNATURES) == set(fns)
    for name, nargs in fns.items():
        assert len(sphkv_lib.SIGNATURES[name][1]) == nargs, name


def test_version_string():
    assert sphkv_lib.version().startswith("sphkv")


def test_workspace_bytes():
    lib = sphkv_lib.load()
    # one (m, l, acc) partial per item, then 16 status bytes
    assert lib.sphkv_decode_paged_workspace_bytes(256, 4, 128) == 256 * (16 + 4 * 128) * 4 + 16
    assert lib.sphkv_decode_paged_workspace_bytes(0, 8, 64) == 16
    assert lib.sphkv_decode_paged_workspace_bytes(4, 3, 128) == -1      # gqa not supported
    assert lib.sphkv_decode_paged_workspace_bytes(4, 4, 96) == -1       # dh not supported
    assert lib.sphkv_decode_paged_workspace_bytes(-1, 4, 128) == -1


def _decode_args(**kw):
    a = dict(pages=None, pages_bytes=0, ptable=None, vslot=None, positions=None, num_rows=0,
             v_pool=None, num_vpages=0, cb1=None, cb2=None, cb3=None, work=None, num_items=0,
             work_start=None, num_seqs=1, num_kv=8, gqa=4, q=None, out=None, workspace=None,
             workspace_bytes=0, dh=128, page_size=16, sm_scale=0.088, rope_theta=5e5, stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(dh=96), "dh must be 64 or 128"),
    (dict(gqa=3), "gqa must be"),
    (dict(page_size=32), "page_size must be 16"),
    (dict(rope_theta=1.0), "rope_theta"),
    (dict(pages_bytes=1970), "multiple of 4"),
    (dict(num_items=8), "workspace too small"),
    (dict(num_items=4, workspace_bytes=10 ** 9), "at least one work item"),
    (dict(num_items=16, workspace_bytes=10 ** 9, work_start=None), "null pointer"),
])
def test_decode_argument_errors(kw, msg):
    lib = sphkv_lib.load()
    rc = lib.sphkv_decode_paged(*_decode_args(**kw))
    assert rc == -1
    assert msg in lib.sphkv_last_error().decode()


def test_decode_rejects_unaddressable_v_pool():
    lib = sphkv_lib.load()
    rc = lib.sphkv_decode_paged(*_decode_args(num_vpages=(1 << 31) + 1, num_items=8, workspace_bytes=10 ** 9))
    assert rc == -1 and "num_vpages" in lib.sphkv_last_error().decode()


def test_decode_status_argument_errors():
    lib = sphkv_lib.load()
    n = ctypes.c_int32(7)
    assert lib.sphkv_decode_paged_status(None, 0, 8, 4, 128, ctypes.byref(n), None) == -1
    assert "does not hold" in lib.sphkv_last_error().decode()
    assert lib.sphkv_decode_paged_status(None, 10 ** 9, 8, 4, 128, None, None) == -1
    assert "null output" in lib.sphkv_last_error().decode()
    # the checked entry validates like sphkv_decode_paged before it launches
    rc = lib.sphkv_decode_paged_checked(*_decode_args(dh=96))
    assert rc == -1 and "dh must be 64 or 128" in lib.sphkv_last_error().decode()
    assert lib.sphkv_decode_paged_checked(*_decode_args(num_seqs=0)) == 0


def test_decode_zero_sequences_is_a_no_op():
    lib = sphkv_lib.load()
    assert lib.sphkv_decode_paged(*_decode_args(num_seqs=0)) == 0
    assert lib.sphkv_last_error().decode() == ""


def test_merge_argument_errors():
    lib = sphkv_lib.load()
    rc = lib.sphkv_decode_merge_partials(None, 0, 8, None, 1, 8, 4, 128, None, None)
    assert rc == -1 and "workspace too small" in lib.sphkv_last_error().decode()
    buf = ctypes.create_string_buffer(8)
    rc = lib.sphkv_decode_merge_partials(buf, 10 ** 9, 8, buf, 1, 8, 4, 128, None, None)
    assert rc == -1 and "null output" in lib.sphkv_last_error().decode()


def test_encode_argument_errors():
    lib = sphkv_lib.load()
    args = [None, 0, None, 0, None, None, None, None, None, None, 4, 8, None, None, None,
            None, 0, None, 0, None, None, 128, 16, None]
    args[21] = 80
    assert lib.sphkv_encode_pages(*args) == -1
    assert "dh must be 64 or 128" in lib.sphkv_last_error().decode()
    args[21] = 128
    assert lib.sphkv_encode_pages(*args) == -1
    assert "null pointer" in lib.sphkv_last_error().decode()


def test_ragged_argument_errors():
    lib = sphkv_lib.load()
    args = [None, 0, None, None, None, 4, None, None, 100, None, 4, 8, None,
            128, 8, 16, 6, 16, None, None]
    args[14] = 7                                   # group_size * groups != dh
    assert lib.sphkv_fused_decode_ragged(*args) == -1
    assert "groups*group_size" in lib.sphkv_last_error().decode()
    args[14] = 8
    args[16] = 9                                   # b_theta
    assert lib.sphkv_fused_decode_ragged(*args) == -1
    assert "b_theta" in lib.sphkv_last_error().decode()
    # the fitted entry: same checks, and the rope model with its fit
    args[16] = 6
    fa = args[:18] + [None, 3] + args[18:]
    assert lib.sphkv_fused_decode_ragged_fitted(*fa) == -1
    assert "rope_model must be 0, 1 or 2" in lib.sphkv_last_error().decode()
    fa[19] = 1                                     # model 1 without a fit
    assert lib.sphkv_fused_decode_ragged_fitted(*fa) == -1
    assert "rope_model" in lib.sphkv_last_error().decode()
    fa[19] = 0
    assert lib.sphkv_fused_decode_ragged_fitted(*fa) == -1
    assert "null pointer" in lib.sphkv_last_error().decode()


def test_rope_table_fit_argument_errors():
    import ctypes
    lib = sphkv_lib.load()
    m = ctypes.c_int32(7)
    assert lib.sphkv_rope_table_fit(None, None, 100, 96, None, ctypes.byref(m), None, None) == -1
    assert "dh must be 64 or 128" in lib.sphkv_last_error().decode()
    assert lib.sphkv_rope_table_fit(None, None, 0, 128, None, ctypes.byref(m), None, None) == -1
    assert "max_pos" in lib.sphkv_last_error().decode()
    assert lib.sphkv_rope_table_fit(None, None, 100, 128, None, ctypes.byref(m), None, None) == -1
    assert "null pointer" in lib.sphkv_last_error().decode()
    assert m.value == 7                            # untouched on error


def _modea_args(**kw):
    a = dict(q=None, cb=None, tG=None, tg=None, th=None, rd=None, rs=None, vp=None, num_pages=0, bt=None,
             bits=None, ctx=None, out=None, part=None, num_q=32, num_kv=8, kv_groups=4, num_tiers=2,
             max_blocks=64, page_size=16, dh=128, G_max=8, cb_max=64, g_max=16, sm_scale=0.088, max_ctx=1024,
             stream=None)
    a.update(kw)
    return list(a.values())


@pytest.mark.parametrize("kw,msg", [
    (dict(dh=96), "dh must be 64 or 128"),
    (dict(num_q=30), "num_q_heads == num_kv_heads * kv_groups"),
    (dict(kv_groups=16, num_q=128), "kv_groups 1..8"),
    (dict(num_tiers=9), "num_tiers must be"),
    (dict(cb_max=512), "bad table geometry"),
    (dict(page_size=24), "page_size must be a multiple of 16"),
    (dict(num_tiers=8, G_max=64, cb_max=256), "LDS"),
    (dict(), "null pointer"),
])
def test_modea_decode_argument_errors(kw, msg):
    lib = sphkv_lib.load()
    assert lib.sphkv_decode_modea(*_modea_args(**kw)) == -1
    assert msg in lib.sphkv_last_error().decode()


def test_modea_decode_empty_is_a_no_op():
    lib = sphkv_lib.load()
    assert lib.sphkv_decode_modea(*_modea_args(max_blocks=0)) == 0
    assert lib.sphkv_decode_modea(*_modea_args(num_kv=0, num_q=0)) == 0


def test_encode_append_argument_errors():
    lib = sphkv_lib.load()
    base = [None] * 8 + [8, 100, 0, 8, 16, 64, 8, 128, 16, 1, None]
    for idx, val, msg in [(15, 300, "dh must be"), (11, 9, "G <= G_max"), (12, 17, "G * g <= dh"),
                          (13, 512, "C <= 256"), (10, 16, "slot must be"), (10, -1, "slot must be"),
                          (9, -5, "negative size"), (10, 0, "null pointer")]:
        args = list(base)
        args[idx] = val
        assert lib.sphkv_encode_append(*args) == -1, msg
        assert msg in lib.sphkv_last_error().decode()
    args = list(base)
    args[8] = 0                                    # no kv heads: nothing to do
    assert lib.sphkv_encode_append(*args) == 0


def test_q_lut_and_logits_argument_errors():
    lib = sphkv_lib.load()
    assert lib.sphkv_q_lut(None, None, None, None, 32, 8, 4, 2, 128, 8, 64, 16, None, None) == -1
    assert "null pointer" in lib.sphkv_last_error().decode()
    assert lib.sphkv_q_lut(None, None, None, None, 33, 8, 4, 2, 128, 8, 64, 16, None, None) == -1
    assert "kv_groups" in lib.sphkv_last_error().decode()
    lg = [None, None, None, None, 10, None, None, None, None, 32, 8, 4, 2, 64, 16, 8, 64, 0.1, 1024, None]
    assert lib.sphkv_logits_lut(*lg) == -1 and "null pointer" in lib.sphkv_last_error().decode()
    lg[16] = 300
    assert lib.sphkv_logits_lut(*lg) == -1 and "bad table geometry" in lib.sphkv_last_error().decode()
    lg[16], lg[18] = 64, 0
    assert lib.sphkv_logits_lut(*lg) == 0


def test_omega_ema_argument_errors():
    lib = sphkv_lib.load()
    assert lib.sphkv_omega_ema(None, None, 130, 2, None, None, 8, 0, 64, 0.9, None) == -1
    assert "kv_groups" in lib.sphkv_last_error().decode()
    assert lib.sphkv_omega_ema(None, None, -1, 2, None, None, 8, 4, 64, 0.9, None) == -1
    assert "negative stride" in lib.sphkv_last_error().decode()
    assert lib.sphkv_omega_ema(None, None, 130, 2, None, None, 8, 4, 64, 0.9, None) == -1
    assert "null pointer" in lib.sphkv_last_error().decode()
    assert lib.sphkv_omega_ema(None, None, 130, 2, None, None, 8, 4, 0, 0.9, None) == 0


def test_noalloc_refuses_work_beyond_its_scratch():
    # the size check runs before any device access
    lib = sphkv_lib.load()
    per_item = lib.sphkv_decode_paged_workspace_bytes(1, 8, 128) - lib.sphkv_decode_paged_workspace_bytes(0, 8, 128)
    n = (8 << 20) // per_item + 1
    args = _decode_args(num_items=n, gqa=8)
    del args[19:21]                                  # no workspace arguments
    assert lib.sphkv_decode_paged_noalloc(*args) == -1
    assert "more than its" in lib.sphkv_last_error().decode()
    args = _decode_args(num_seqs=0)
    del args[19:21]
    assert lib.sphkv_decode_paged_noalloc(*args) == 0


def test_decode_plan_argument_errors():
    import ctypes
    lib = sphkv_lib.load()
    h = ctypes.c_void_p(123)
    # (pages, bytes, ptable, vslot, positions, rows, v_pool, vpages, cb1..3, work, items, work_start,
    #  seqs, kv, gqa, workspace, ws_bytes, dh, page_size, sm_scale, theta, plan_out)
    args = [None, 0, None, None, None, 0, None, 0, None, None, None, None, 8, None, 1, 8, 4, None, 1 << 20,
            96, 16, 0.1, 500000.0, ctypes.byref(h)]
    assert lib.sphkv_decode_plan_create(*args) == -1
    assert "dh must be 64 or 128" in lib.sphkv_last_error().decode()
    assert h.value is None                         # no plan on error
    args[19] = 128
    args[14] = 0                                   # no sequence: nothing a plan could run
    assert lib.sphkv_decode_plan_create(*args) == -1
    args[14] = 1
    assert lib.sphkv_decode_plan_create(*args) == -1
    assert "null pointer" in lib.sphkv_last_error().decode()
    args[-1] = None
    assert lib.sphkv_decode_plan_create(*args) == -1
    assert "plan_out" in lib.sphkv_last_error().decode()
    assert lib.sphkv_decode_plan_run(None, None, None, None) == -1
    lib.sphkv_decode_plan_destroy(None)            # a no-op


def test_decode_runner_closure_keeps_its_plan_alive(monkeypatch):
    # the raw() form of a bound decode holds its runner, so the C plan cannot
    # be destroyed while the closure exists (a runner built and dropped in one
    # expression, DecodeRunner(...).raw(), must stay usable); built here with
    # stand-in addresses: plan creation checks arguments and touches no memory
    import ctypes
    import gc
    import weakref
    import sphkv_ops as ops
    lib = sphkv_lib.load()
    h = ctypes.c_void_p()
    fake = 1 << 20                                    # non-null stand-in address, never dereferenced
    rc = lib.sphkv_decode_plan_create(fake, 1024, fake, fake, fake, 8, fake, 8, fake, None, None, fake, 8, fake,
                                      1, 8, 4, fake, 1 << 20, 128, 16, 0.1, 500000.0, ctypes.byref(h))
    assert rc == 0 and h.value
    monkeypatch.setattr(ops, "_stream", lambda: 0)    # (no device here: the default stream's handle)
    r = object.__new__(ops.DecodeRunner)
    r._plan, r._run = h.value, lib.sphkv_decode_plan_run
    alive = weakref.ref(r)
    fn = r.raw()
    del r
    gc.collect()
    assert alive() is not None                        # held by fn
    del fn
    gc.collect()
    assert alive() is None                            # and released with it (its plan destroyed)


# ------------------------------------------------- decode step and its plan --
_FAKE = 1 << 20                                      # non-null stand-in address, never dereferenced


def _step_plan_args(**kw):
    """sphkv_step_plan_create's arguments for 1 sequence x 8 kv heads at dh 128,
    gqa 4, 8 items, room for 2 decode pages per (seq, head); plan_out last."""
    d = dict(pages=_FAKE, pages_bytes=1 << 16, ptable=_FAKE, vslot=_FAKE, positions=_FAKE, num_rows=8,
             v_pool=_FAKE, num_vpages=64, cb1=_FAKE, cb2=None, cb3=_FAKE, work=_FAKE, num_items=8,
             work_start=_FAKE, num_seqs=1, num_kv=8, gqa=4, stg_r=_FAKE, stg_code=_FAKE, stg_v=_FAKE,
             stg_pos=_FAKE, tail_state=_FAKE, dec_byte0=4096, dec_vpage0=8, dec_cap=2, staged=0, flushed=0,
             step_parity=0, workspace=_FAKE, workspace_bytes=1 << 20, dh=128, page_size=16, sm_scale=0.1,
             rope_theta=500000.0)
    d.update(kw)
    return list(d.values())


@pytest.mark.parametrize("kw, msg", [
    (dict(staged=16), "staged must be 0..15"),
    (dict(flushed=3), "flushed 0..dec_cap"),
    (dict(dec_byte0=4100), "16-byte aligned"),
    (dict(dec_cap=1000), "leaves the byte pool"),
    (dict(dec_vpage0=60), "V slots leave the V pool"),
    (dict(cb3=None), "tier-3 codebook is required"),
    (dict(stg_v=None), "null pointer"),
    (dict(num_seqs=0), "num_seqs must be > 0"),
    (dict(num_items=7), "one work item per (seq, head)"),
    (dict(workspace_bytes=1024), "workspace too small"),
    (dict(step_parity=2), "step_parity must be 0 or 1"),
    (dict(gqa=3), "gqa must be"),
])
def test_step_plan_argument_errors(kw, msg):
    lib = sphkv_lib.load()
    h = ctypes.c_void_p()
    assert lib.sphkv_step_plan_create(*_step_plan_args(**kw), ctypes.byref(h)) == -1
    assert msg in lib.sphkv_last_error().decode()
    assert h.value is None


def test_step_plan_counts_and_capacity():
    # plan creation checks arguments only; a run that would need a decode
    # page past dec_cap, or whose mode or inputs are bad, fails before any
    # launch and leaves the host's counts unchanged
    lib = sphkv_lib.load()
    h = ctypes.c_void_p()
    assert lib.sphkv_step_plan_create(*_step_plan_args(staged=15, flushed=2, step_parity=1), ctypes.byref(h)) == 0
    a, b, p = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    assert lib.sphkv_step_plan_counts(h, ctypes.byref(a), ctypes.byref(b), ctypes.byref(p)) == 0
    assert (a.value, b.value, p.value) == (15, 2, 1)
    for mode in (2, 3):                                # appending: the 16th token needs a third page
        assert lib.sphkv_step_plan_run(h, _FAKE, _FAKE, 0, _FAKE, _FAKE, _FAKE, mode, None) == -1
        assert "no decode-page slot left" in lib.sphkv_last_error().decode()
    for mode in (0, 4):
        assert lib.sphkv_step_plan_run(h, _FAKE, _FAKE, 0, _FAKE, _FAKE, _FAKE, mode, None) == -1
        assert "mode must be" in lib.sphkv_last_error().decode()
    assert lib.sphkv_step_plan_run(h, _FAKE, None, 0, _FAKE, _FAKE, _FAKE, 3, None) == -1
    assert "null pointer" in lib.sphkv_last_error().decode()
    assert lib.sphkv_step_plan_run(h, None, _FAKE, 0, _FAKE, _FAKE, _FAKE, 1, None) == -1   # decode needs q
    assert lib.sphkv_step_plan_counts(h, ctypes.byref(a), ctypes.byref(b), ctypes.byref(p)) == 0
    assert (a.value, b.value, p.value) == (15, 2, 1)
    lib.sphkv_step_plan_destroy(h)
    assert lib.sphkv_step_plan_run(None, _FAKE, _FAKE, 0, _FAKE, _FAKE, _FAKE, 3, None) == -1
    assert lib.sphkv_step_plan_counts(None, ctypes.byref(a), ctypes.byref(b), ctypes.byref(p)) == -1
    lib.sphkv_step_plan_destroy(None)                  # a no-op


def _step_args(**kw):
    """sphkv_decode_step's arguments (shapes as _step_plan_args), stream last."""
    d = dict(pages=_FAKE, pages_bytes=1 << 16, ptable=_FAKE, vslot=_FAKE, positions=_FAKE, num_rows=8,
             v_pool=_FAKE, num_vpages=64, cb1=_FAKE, cb2=None, cb3=_FAKE, work=_FAKE, num_items=8,
             work_start=_FAKE, num_seqs=1, num_kv=8, gqa=4, q=_FAKE, k_new=_FAKE, k_is_fp32=0, v_new=_FAKE,
             cur_pos=_FAKE, stg_r=_FAKE, stg_code=_FAKE, stg_v=_FAKE, stg_pos=_FAKE, tail_state=_FAKE,
             dec_byte0=4096, dec_vpage0=8, dec_cap=2, append=1, step_parity=0, out=_FAKE, workspace=_FAKE,
             workspace_bytes=1 << 20, dh=128, page_size=16, sm_scale=0.1, rope_theta=500000.0, stream=None)
    d.update(kw)
    return list(d.values())


@pytest.mark.parametrize("kw, msg", [
    (dict(append=2), "append must be 0 or 1"),
    (dict(step_parity=-1), "step_parity must be 0 or 1"),
    (dict(pages_bytes=(1 << 16) + 2), "multiple of 4"),
    (dict(rope_theta=1.0), "rope_theta must be > 1"),
    (dict(k_new=None), "null pointer"),
    (dict(out=None), "null pointer"),
    (dict(dec_cap=1000), "leaves the byte pool"),
    (dict(page_size=128), "page_size must be 16"),
])
def test_decode_step_argument_errors(kw, msg):
    lib = sphkv_lib.load()
    assert lib.sphkv_decode_step(*_step_args(**kw)) == -1
    assert msg in lib.sphkv_last_error().decode()


def test_decode_step_and_append_with_no_sequence_are_no_ops():
    lib = sphkv_lib.load()
    assert lib.sphkv_decode_step(*_step_args(num_seqs=0, q=None, k_new=None, out=None)) == 0
    # (pages, bytes, positions, rows, v_pool, vpages, cb3, work, items, work_start, seqs, kv, k_new,
    #  k_is_fp32, v_new, cur_pos, stg_r, stg_code, stg_v, stg_pos, tail_state, dec_byte0, dec_vpage0,
    #  dec_cap, step_parity, dh, page_size, stream)
    app = [_FAKE, 1 << 16, _FAKE, 8, _FAKE, 64, _FAKE, _FAKE, 8, _FAKE, 0, 8, None, 0, None, None, _FAKE, _FAKE,
           _FAKE, _FAKE, _FAKE, 4096, 8, 2, 0, 128, 16, None]
    assert lib.sphkv_decode_append(*app) == 0
    app[10] = 1
    assert lib.sphkv_decode_append(*app) == -1         # a sequence, no k_new
    assert "null pointer" in lib.sphkv_last_error().decode()
    app[12], app[14], app[15] = _FAKE, _FAKE, _FAKE
    app[6] = None
    assert lib.sphkv_decode_append(*app) == -1
    assert "tier-3 codebook is required" in lib.sphkv_last_error().decode()
    app[6] = _FAKE
    app[24] = 5
    assert lib.sphkv_decode_append(*app) == -1
    assert "step_parity must be 0 or 1" in lib.sphkv_last_error().decode()


def test_tail_relayout_argument_errors():
    lib = sphkv_lib.load()
    # (row_start, num_sh, num_rows, ptable, vslot, positions, dec_cap, dec_byte0, dec_vpage0, dh,
    #  ptable_d, vslot_d, positions_d, stream)
    args = [_FAKE, 8, 100, _FAKE, _FAKE, _FAKE, 4, 4096, 100, 128, _FAKE, _FAKE, _FAKE, None]
    bad = [(dict(i=9, v=96), "dh must be 64 or 128"), (dict(i=7, v=4100), "16-byte aligned"),
           (dict(i=6, v=-1), "bad size"), (dict(i=6, v=1 << 28), "outgrows int32"),
           (dict(i=10, v=None), "null pointer")]
    for b, msg in bad:
        a = list(args)
        a[b["i"]] = b["v"]
        assert lib.sphkv_tail_relayout(*a) == -1
        assert msg in lib.sphkv_last_error().decode()
    a = list(args)
    a[1], a[2], a[3], a[4], a[5] = 0, 0, None, None, None
    assert lib.sphkv_tail_relayout(*a) == 0            # nothing to lay out
