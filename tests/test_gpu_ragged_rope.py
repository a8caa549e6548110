"""GPU: fused_decode_ragged with the caller's RoPE tables fitted once
(sphkv_rope_table_fit) and the phases formed in the kernel.

The reference's callers pass one pair of tables, built by the model's rotary
embedding (spherical_kv_pipeline.py:1591-1610; HF: fp32 inv_freq times the
fp32 position, then cos / sin), to every call (:1102-1125).  Checked here:

* the fit's model on tables of known construction: exact fp64 angles
  (sphkv_format.rope_tables) -> 1; transformers' LlamaRotaryEmbedding, plain
  and with Llama-3.1 scaling, and an fp32-angle construction of our own -> 2;
  bf16-rounded tables, one entry moved by 1e-4 in the last row, or one row
  whose halves differ -> 0 (read as given);
* logits of the fitted path against the fp64 oracle over the same tables
  (within 2e-4, as the table path) and against the table path itself (within
  2e-5), positions up to 131K;
* the fit is cached per tensor pair and version: a second call does not fit
  again, an in-place change of a table does;
* a fit of another model passed to the C entry makes every logit NaN.
"""
import ctypes

import numpy as np
import pytest
import torch

import fused_decode
import oracle
from oracle import paging
import sphkv_format as fmt
import sphkv_lib
import sphkv_synth as synth
from gpu_helpers import log, max_err

pytestmark = pytest.mark.gpu
THETA = 500000.0


def _fp32_angle_tables(max_pos, dh, theta, dev):
    """cos / sin of fl32(fl32(pos) * inv32), inv32 = fp32 theta^(-2j/dh)."""
    return synth.hf_rope_tables(max_pos, dh, theta, dev)


def _hf_tables(max_pos, dh, dev, llama3=False):
    """The tables as the reference builds them: the rotary embedding of a
    Llama config at positions 0 .. max_pos - 1 (fp32)."""
    from transformers import LlamaConfig
    from transformers.models.llama.modeling_llama import LlamaRotaryEmbedding
    kw = dict(hidden_size=32 * dh, num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=131072)
    if llama3:
        kw["rope_parameters"] = {"rope_type": "llama3", "rope_theta": THETA, "factor": 8.0, "low_freq_factor": 1.0,
                                 "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    else:
        kw["rope_theta"] = THETA
    rot = LlamaRotaryEmbedding(config=LlamaConfig(**kw)).to(dev)
    pos = torch.arange(max_pos, device=dev).unsqueeze(0)
    cos, sin = rot(torch.zeros(1, 1, 1, dh, device=dev, dtype=torch.float32), pos)
    return cos[0].float().contiguous(), sin[0].float().contiguous()


def _tier_pages(tid, dh, num_kv, L, max_pos, page_size, seed):
    """num_kv heads of L tokens at sorted distinct positions < max_pos, encoded
    by the oracle into pages laid out back to back (one tier)."""
    rng = np.random.default_rng(seed)
    g, b = fmt.TIER_GEOMETRY[tid]
    G = dh // g
    cbs = synth.make_codebooks(rng, num_kv, dh, [tid])[tid]
    buf, ptab, heads, pos = [], [], [], []
    base = 0
    for h in range(num_kv):
        K = (rng.standard_normal((L, dh)) * np.exp(rng.normal(0, 0.5, dh))).astype(np.float16)
        idx = np.sort(rng.choice(max_pos, size=L, replace=False))
        counts = [min(page_size, L - s) for s in range(0, L, page_size)]
        rows = paging.page_offsets(tid, counts, dh).astype(np.int64) + base
        for ci, s0 in enumerate(range(0, L, page_size)):
            n = counts[ci]
            r, codes = oracle.encode_groups(K[s0:s0 + n].astype(np.float32), cbs[h])
            buf.append(oracle.build_page(r, codes, tid, b))
            pp = np.full(page_size, -1, np.int32)
            pp[:n] = idx[s0:s0 + n]
            pos.append(pp)
            heads.append(h)
        ptab.append(rows)
        base += sum(x.size for x in buf[len(buf) - len(counts):])
    return dict(pages=np.concatenate(buf), ptable=np.concatenate(ptab).astype(np.int32),
                heads=np.asarray(heads, np.int32), pos=np.concatenate(pos).astype(np.int32),
                cb=cbs.reshape(num_kv * G, 2 ** b, g), G=G, g=g, b=b)


def _ragged(d, cos_t, sin_t, q, grp, num_kv, dh, page_size, gpu):
    t = lambda x: torch.as_tensor(x, device=gpu)
    return fused_decode.fused_decode_ragged(
        t(d["pages"]), t(d["ptable"]), t(d["heads"]), t(d["pos"]), cos_t, sin_t, t(q), grp, num_kv, t(d["cb"]),
        dh, d["G"], d["g"], d["b"], page_size)


@pytest.mark.parametrize("kind,dh,want", [
    ("exact", 128, 1), ("exact", 64, 1), ("fp32", 128, 2), ("hf", 128, 2), ("hf_llama3", 128, 2), ("hf", 64, 2),
    ("bf16", 128, 0), ("moved", 128, 0), ("halves", 128, 0)])
def test_rope_fit_model_of_known_tables(gpu, kind, dh, want):
    max_pos = 131072 + 64
    if kind in ("exact", "moved", "halves"):
        c, s = fmt.rope_tables(max_pos, dh, THETA)
        c, s = torch.as_tensor(c, device=gpu), torch.as_tensor(s, device=gpu)
        if kind == "moved":
            c[max_pos - 1, 5] += 1e-4
        if kind == "halves":
            c[777, dh // 2 + 3] = torch.nextafter(c[777, dh // 2 + 3], torch.tensor(2.0, device=gpu))
    elif kind == "fp32":
        c, s = _fp32_angle_tables(max_pos, dh, THETA, gpu)
    elif kind.startswith("hf"):
        c, s = _hf_tables(max_pos, dh, gpu, llama3=kind == "hf_llama3")
    else:
        c, s = _fp32_angle_tables(max_pos, dh, THETA, gpu)
        c, s = c.bfloat16().float(), s.bfloat16().float()
    model, dev_exact, dev_fp32 = fused_decode.rope_fit_info(c, s)
    log(f"  {kind} dh {dh}: model {model}, deviation exact {dev_exact:.3e}, fp32 {dev_fp32:.3e}")
    assert model == want
    if want == 1:
        assert dev_exact <= 2.0 ** -20
    if want == 2:
        assert dev_fp32 <= 2.0 ** -20 and dev_exact > 2.0 ** -20


@pytest.mark.parametrize("kind,tid,dh,grp,num_kv,page_size", [
    ("exact", 1, 128, 4, 2, 16), ("hf", 1, 128, 4, 2, 16), ("hf_llama3", 2, 128, 8, 2, 128),
    ("fp32", 3, 64, 4, 3, 32), ("hf", 2, 64, 2, 2, 16), ("bf16", 1, 128, 4, 2, 16)])
def test_ragged_fitted_matches_oracle_and_table_path(gpu, kind, tid, dh, grp, num_kv, page_size):
    max_pos = 131072 + 64
    if kind == "exact":
        c, s = (torch.as_tensor(x, device=gpu) for x in fmt.rope_tables(max_pos, dh, THETA))
    elif kind == "fp32":
        c, s = _fp32_angle_tables(max_pos, dh, THETA, gpu)
    elif kind == "bf16":
        c, s = _fp32_angle_tables(max_pos, dh, THETA, gpu)
        c, s = c.bfloat16().float(), s.bfloat16().float()
    else:
        c, s = _hf_tables(max_pos, dh, gpu, llama3=kind == "hf_llama3")
    d = _tier_pages(tid, dh, num_kv, 300, max_pos, page_size, seed=900 + tid + dh + grp)
    q = np.random.default_rng(5).standard_normal((num_kv * grp, dh)).astype(np.float32)
    model = fused_decode.rope_fit_info(c, s)[0]
    got = _ragged(d, c, s, q, grp, num_kv, dh, page_size, gpu).cpu().numpy()
    fused_decode.use_rope_fit = False
    try:
        tab = _ragged(d, c, s, q, grp, num_kv, dh, page_size, gpu).cpu().numpy()
    finally:
        fused_decode.use_rope_fit = True
    want = oracle.ragged_logits(d["pages"], d["ptable"], d["heads"], d["pos"], c.cpu().numpy(), s.cpu().numpy(),
                                q, grp, d["cb"], dh, d["G"], d["g"], d["b"], page_size)
    fin = np.isfinite(want)
    assert fin.sum() == num_kv * 300 * grp
    assert (np.isneginf(got) == ~fin).all() and (np.isneginf(tab) == ~fin).all()
    e_or, e_tab = max_err(got[fin], want[fin]), max_err(got[fin], tab[fin])
    log(f"  {kind} tier {tid} dh {dh} grp {grp}: model {model}, vs oracle {e_or:.3e}, vs table path {e_tab:.3e}")
    assert e_or < 2e-4 and e_tab < 2e-5


def test_rope_fit_is_cached_per_table_version(gpu):
    dh, grp, num_kv, max_pos = 128, 4, 2, 9000
    c, s = _fp32_angle_tables(max_pos, dh, THETA, gpu)
    d = _tier_pages(1, dh, num_kv, 200, max_pos, 16, seed=31)
    q = np.random.default_rng(6).standard_normal((num_kv * grp, dh)).astype(np.float32)
    n0 = fused_decode.fit_calls
    a = _ragged(d, c, s, q, grp, num_kv, dh, 16, gpu)
    b = _ragged(d, c, s, q, grp, num_kv, dh, 16, gpu)
    assert fused_decode.fit_calls == n0 + 1 and torch.equal(a, b)
    assert fused_decode.rope_fit_info(c, s)[0] == 2
    # an in-place change (version bump): fitted again, and now read as given
    row = int(d["pos"][d["pos"] >= 0][7])
    c[row, :] = c[row, :] * 0.5
    got = _ragged(d, c, s, q, grp, num_kv, dh, 16, gpu).cpu().numpy()
    assert fused_decode.fit_calls == n0 + 2 and fused_decode.rope_fit_info(c, s)[0] == 0
    want = oracle.ragged_logits(d["pages"], d["ptable"], d["heads"], d["pos"], c.cpu().numpy(), s.cpu().numpy(),
                                q, grp, d["cb"], dh, d["G"], d["g"], d["b"], 16)
    fin = np.isfinite(want)
    assert max_err(got[fin], want[fin]) < 2e-4
    # a new pair of tensors with equal contents is fitted on its own
    c2, s2 = c.clone(), s.clone()
    _ragged(d, c2, s2, q, grp, num_kv, dh, 16, gpu)
    assert fused_decode.fit_calls == n0 + 3


def test_fit_of_another_model_gives_nan(gpu):
    # the C entry checks the fit it is handed against the model it is told
    dh, grp, num_kv, max_pos = 128, 4, 2, 5000
    c, s = (torch.as_tensor(x, device=gpu) for x in fmt.rope_tables(max_pos, dh, THETA))
    lib = sphkv_lib.load()
    fit = torch.empty(fused_decode.ROPE_FIT_BYTES, dtype=torch.uint8, device=gpu)
    m = ctypes.c_int32(-1)
    assert lib.sphkv_rope_table_fit(c.data_ptr(), s.data_ptr(), max_pos, dh, fit.data_ptr(), ctypes.byref(m), None,
                                    sphkv_lib.current_stream()) == 0
    assert m.value == 1
    d = _tier_pages(1, dh, num_kv, 64, max_pos, 16, seed=32)
    t = lambda x: torch.as_tensor(x, device=gpu)
    pages, ptable, heads, pos, cb = t(d["pages"]), t(d["ptable"]), t(d["heads"]), t(d["pos"]), t(d["cb"])
    q = t(np.ones((num_kv * grp, dh), np.float32))
    P = int(ptable.shape[0])
    out = torch.zeros((grp, P * 16), dtype=torch.float32, device=gpu)
    for model, nan in ((1, False), (2, True)):
        rc = lib.sphkv_fused_decode_ragged_fitted(
            pages.data_ptr(), pages.numel(), ptable.data_ptr(), heads.data_ptr(), pos.data_ptr(), P, c.data_ptr(),
            s.data_ptr(), max_pos, q.data_ptr(), grp, num_kv, cb.data_ptr(), dh, d["G"], d["g"], d["b"], 16,
            fit.data_ptr(), model, out.data_ptr(), sphkv_lib.current_stream())
        assert rc == 0
        torch.cuda.synchronize()
        assert bool(torch.isnan(out).all()) == nan
        assert nan or bool(torch.isfinite(out[:, :16]).any())
