"""GPU parity of the opaque operators, the compiled facades and StaticCache decode.

Mirrors the reference's operator tests (tests/test_h100_torch_ops.py:317-512)
and adds numerical parity, which the reference checks only through its
adapters:

* the row-preparation kernel at head_dim 256 and 512 with bf16 tables (the
  layers' q / k / v RMSNorm + RoPE) against the reference's torch operations
  (oracle ``reference_kv_prep``: at least 99.5% bit-identical, every element
  within one bf16 ulp of its terms), written into strided views;
* the prepared-tensor operators bitwise equal to the adapters they wrap;
* the whole-layer operators against the installed Transformers
  ``Gemma4TextAttention`` running this library's attention backend (same
  arithmetic apart from the preparation kernel: rel-Frobenius < 3e-3) and
  against an fp64 composition of oracle pieces (rel-Frobenius < 1e-2, LSE in
  the M1 envelope);
* StaticCache decode against the same fp64 composition over the cache, the
  exact cache mutation (new slot, sliding roll, untouched slots bitwise) and
  the facades' counters over steps that cross the sliding window's capacity.
"""

from __future__ import annotations

import pytest
import torch

from oracle.envelope import GLOBAL_LSE_ATOL, LOCAL_LSE_ATOL, rel_frobenius
from oracle.kv_prep import reference_kv_prep
from g4_testutil import oracle_fwd_bwd

pytestmark = pytest.mark.gpu
DEV = "cuda"
mg = pytest.importorskip("transformers.models.gemma4.modeling_gemma4")
cache_utils = pytest.importorskip("transformers.cache_utils")

FAMILY = {"local": dict(layer=0, d=256, hkv=16, window=1024),
          "global": dict(layer=5, d=512, hkv=4, window=None)}


def _ops():
    from gemma4_fa4_amd import torch_ops

    return torch_ops


def _config():
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig

    return Gemma4TextConfig(hidden_size=5376, num_attention_heads=32, num_key_value_heads=16,
                            head_dim=256, global_head_dim=512, num_global_key_value_heads=4,
                            attention_k_eq_v=True, sliding_window=1024, num_hidden_layers=60,
                            hidden_size_per_layer_input=0, vocab_size_per_layer_input=0,
                            max_position_embeddings=262144)


_MODULES: dict = {}


def _module(family):
    """A 31B-geometry Transformers attention layer with seeded weights (cached per family)."""
    if family not in _MODULES:
        cfg = _config()
        torch.manual_seed(11 if family == "local" else 12)
        with torch.device(DEV):
            m = mg.Gemma4TextAttention(cfg, FAMILY[family]["layer"]).to(torch.bfloat16).eval()
            for norm in (m.q_norm, m.k_norm):
                norm.weight.data = (torch.rand_like(norm.weight, dtype=torch.float32) + 0.5) \
                    .to(torch.bfloat16)
        _MODULES[family] = (cfg, m, mg.Gemma4TextRotaryEmbedding(cfg).to(DEV))
    return _MODULES[family]


def _rope(family, positions):
    cfg, m, rot = _module(family)
    kind = "sliding_attention" if family == "local" else "full_attention"
    x = torch.zeros(1, 1, 1, dtype=torch.bfloat16, device=DEV)
    return rot(x, positions.to(DEV), kind)


def _hidden(seed, s):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(1, s, 5376, generator=g).to(torch.bfloat16).to(DEV)


def _weights(family):
    from gemma4_fa4_amd.facades import layer_weights

    return layer_weights(_module(family)[1])


def _ulp_check(got, want, label, mag=None, min_equal=0.995):
    got, want = got.float().cpu(), want.float().cpu()
    lim = (want.abs() if mag is None else mag) * 2.0 ** -7 + 1e-6
    bad = int(((got - want).abs() > lim).sum())
    equal = (got == want).float().mean().item()
    assert bad == 0, f"{label}: {bad} elements beyond one bf16 ulp"
    assert equal >= min_equal, f"{label}: only {equal:.4f} bit-identical"


def _rope_magnitude(kn, cos, sin):
    """|kn_i cos_i| + |kn_partner sin_i| (full-width rotation) of (B, H, S, D) rows."""
    kn = kn.float()
    half = kn.shape[-1] // 2
    partner = torch.cat((kn[..., half:], kn[..., :half]), dim=-1).abs()
    return kn.abs() * cos.float()[:, None].abs() + partner * sin.float()[:, None].abs()


def _prepare_reference(src_bshd, weight, cos, sin, *, value=False):
    """The layers' RMSNorm(+RoPE) in the reference's torch operations, on the CPU (BHSD)."""
    src = src_bshd.transpose(1, 2).cpu()
    w = weight.cpu()
    k, v = reference_kv_prep(src, k_norm_weight=w, cos=cos.cpu(), sin=sin.cpu(),
                             partial_rotary_factor=1.0)
    if value:
        return v
    kn, _ = reference_kv_prep(src, k_norm_weight=w, cos=cos.cpu(), sin=sin.cpu(),
                              partial_rotary_factor=0.0)
    return k, _rope_magnitude(kn, cos.cpu(), sin.cpu())


# --------------------------------------------------------------------------
# row preparation kernel, head_dim 256 / 512, bf16 tables
# --------------------------------------------------------------------------


@pytest.mark.parametrize("family,heads,s", [("local", 32, 77), ("local", 16, 300),
                                            ("global", 32, 65), ("global", 4, 300)])
def test_row_preparation_matches_the_reference_operations(family, heads, s):
    from gemma4_fa4_amd.kv_prep import prepare_rows_into

    d = FAMILY[family]["d"]
    g = torch.Generator().manual_seed(s + heads)
    src = (torch.randn(1, s, heads, d, generator=g) * 3).to(torch.bfloat16).to(DEV)
    w = (torch.rand(d, generator=g) + 0.5).to(torch.bfloat16).to(DEV)
    cos, sin = _rope(family, torch.arange(s)[None] + 5)
    k = torch.empty_like(src)
    v = torch.empty_like(src)
    prepare_rows_into(src.transpose(1, 2), weight=w, cos=cos, sin=sin, rotary_dim=d,
                      k=k.transpose(1, 2), v=v.transpose(1, 2))
    torch.cuda.synchronize()
    rk, mag = _prepare_reference(src, w, cos, sin)
    rv = _prepare_reference(src, w, cos, sin, value=True)
    _ulp_check(k.transpose(1, 2), rk, f"{family} K", mag=mag)
    _ulp_check(v.transpose(1, 2), rv, f"{family} V")


def test_row_preparation_writes_only_its_views():
    from gemma4_fa4_amd.kv_prep import prepare_rows_into

    g = torch.Generator().manual_seed(3)
    cache_k = torch.randn(1, 16, 40, 256, generator=g).to(torch.bfloat16).to(DEV)
    cache_v = torch.randn(1, 16, 40, 256, generator=g).to(torch.bfloat16).to(DEV)
    before_k, before_v = cache_k.clone(), cache_v.clone()
    src = torch.randn(1, 1, 16, 256, generator=g).to(torch.bfloat16).to(DEV)
    w = torch.ones(256, dtype=torch.bfloat16, device=DEV)
    cos, sin = _rope("local", torch.tensor([[17]]))
    prepare_rows_into(src.transpose(1, 2), weight=w, cos=cos, sin=sin, rotary_dim=256,
                      k=cache_k[:, :, 17:18])
    prepare_rows_into(src.transpose(1, 2), weight=w, v=cache_v[:, :, 9:10])
    torch.cuda.synchronize()
    keep = torch.ones(40, dtype=torch.bool)
    keep[17] = False
    assert torch.equal(cache_k[:, :, keep], before_k[:, :, keep])
    keep = torch.ones(40, dtype=torch.bool)
    keep[9] = False
    assert torch.equal(cache_v[:, :, keep], before_v[:, :, keep])
    rk, mag = _prepare_reference(src, w, cos, sin)
    _ulp_check(cache_k[:, :, 17:18], rk, "slot K", mag=mag, min_equal=0.99)
    _ulp_check(cache_v[:, :, 9:10], _prepare_reference(src, w, cos, sin, value=True), "slot V",
               min_equal=0.99)


# --------------------------------------------------------------------------
# prepared-tensor operators
# --------------------------------------------------------------------------


def _prepared(family, s, seed=0):
    f = FAMILY[family]
    g = torch.Generator().manual_seed(seed + s)
    sd = f["d"] ** -0.25
    q = (torch.randn(1, 32, s, f["d"], generator=g) * sd).to(torch.bfloat16).to(DEV)
    k = (torch.randn(1, f["hkv"], s, f["d"], generator=g) * sd).to(torch.bfloat16).to(DEV)
    v = torch.randn(1, f["hkv"], s, f["d"], generator=g).to(torch.bfloat16).to(DEV)
    pos = torch.arange(s, device=DEV).unsqueeze(0)
    return q, k, v, pos, torch.zeros_like(pos)


@pytest.mark.parametrize("family", ["local", "global"])
@pytest.mark.parametrize("s", [1, 300, 1024])
def test_prepared_operators_equal_their_adapters(family, s):
    import gemma4_fa4_amd as g4

    ops = _ops()
    op = ops.local_fwd if family == "local" else ops.global_fwd
    adapter = g4.fa4_local_text_forward if family == "local" else g4.fa4_global_text_forward
    q, k, v, pos, packed = _prepared(family, s)
    with torch.inference_mode():
        out, lse = op(q, k, v, pos, packed)
        ref_o, ref_l = adapter(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    torch.cuda.synchronize()
    assert out.shape == (1, s, 32, q.shape[-1]) and lse.shape == (1, 32, s)
    assert out.dtype == torch.bfloat16 and lse.dtype == torch.float32
    assert torch.equal(out, ref_o) and torch.equal(lse, ref_l)
    pointers = {t.untyped_storage().data_ptr() for t in (q, k, v, out, lse)}
    assert len(pointers) == 5


@pytest.mark.parametrize("family", ["local", "global"])
def test_opcheck_passes_the_prepared_operator_contract(family):
    ops = _ops()
    op = ops.local_fwd if family == "local" else ops.global_fwd
    result = torch.library.opcheck(op, _prepared(family, 1))
    assert set(result.values()) == {"SUCCESS"}


def test_prepared_operators_reject_what_the_reference_rejects():
    ops = _ops()
    q, k, v, pos, packed = _prepared("local", 2)
    from gemma4_fa4_amd.errors import UnsupportedMI355XPath

    with torch.inference_mode():
        with pytest.raises(UnsupportedMI355XPath, match="arange"):
            ops.local_fwd(q, k, v, torch.tensor([[0, 0]], device=DEV), packed)
        with pytest.raises(ValueError, match="distinct storage"):
            ops.local_fwd(q, k, k, pos, packed)
        with pytest.raises(ValueError, match="distinct storage"):
            ops.local_fwd(q, q[:, :16], v, pos, packed)
        with pytest.raises(UnsupportedMI355XPath, match="derived exactly"):
            ops.local_fwd(q, k, v, pos, torch.tensor([[0, 1]], device=DEV))
        for bad in (torch.empty(1, dtype=torch.int64, device=DEV),
                    torch.empty((1, 2), dtype=torch.float32, device=DEV)):
            with pytest.raises(ValueError, match="position_ids"):
                ops.local_fwd(q, k, v, bad, packed)
        for bad in (packed[0], packed.float()):
            with pytest.raises(ValueError, match="packed_sequence_ids"):
                ops.local_fwd(q, k, v, pos, bad)
        with pytest.raises(ValueError, match="rank-4"):
            ops.local_fwd(q[0], k, v, pos, packed)
        with pytest.raises(ValueError, match="BF16"):
            ops.local_fwd(q.float(), k, v, pos, packed)
        with pytest.raises(ValueError, match="geometry"):
            ops.local_fwd(q[:, :31], k, v, pos, packed)
        for s in (0, 1025):
            qs, ks, vs, ps, pk = (torch.empty(1, 32, s, 256, dtype=torch.bfloat16, device=DEV),
                                  torch.empty(1, 16, s, 256, dtype=torch.bfloat16, device=DEV),
                                  torch.empty(1, 16, s, 256, dtype=torch.bfloat16, device=DEV),
                                  torch.arange(s, device=DEV)[None],
                                  torch.zeros(1, s, dtype=torch.int64, device=DEV))
            with pytest.raises(UnsupportedMI355XPath, match="1 <= S <= 1024"):
                ops.local_fwd(qs, ks, vs, ps, pk)
        q1, k1, v1, p1, pk1 = _prepared("local", 1)
        misaligned = torch.empty((1, 32, 1, 257), dtype=torch.bfloat16, device=DEV)[..., 1:]
        with pytest.raises(ValueError, match="16-byte aligned"):
            ops.local_fwd(misaligned, k1, v1, p1, pk1)
    q.requires_grad_(True)
    with torch.no_grad(), pytest.raises(UnsupportedMI355XPath, match="requires_grad"):
        ops.local_fwd(q, k, v, pos, packed)


# --------------------------------------------------------------------------
# whole-layer operators and the layer facade
# --------------------------------------------------------------------------


def _oracle_attention_out(family, q_bshd, k_bshd, v_bshd, o_weight):
    """fp64 attention of prepared (CPU, bf16) q / k / v, then the fp64 output projection."""
    f = FAMILY[family]
    sq, sk = q_bshd.shape[1], k_bshd.shape[1]
    cu_q = torch.tensor([0, sq], dtype=torch.int32)
    cu_k = torch.tensor([0, sk], dtype=torch.int32)
    o, lse = oracle_fwd_bwd(q_bshd[0], k_bshd[0], v_bshd[0], cu_q, cu_k, window=f["window"])[:2]
    out = o.reshape(sq, -1).double() @ o_weight.double().cpu().T
    return out[None], lse[None]


def _layer_reference(family, h, cos, sin, weights):
    f = FAMILY[family]
    lin = torch.nn.functional.linear
    d, hkv = f["d"], f["hkv"]
    s = h.shape[1]
    qs = lin(h, weights[0]).view(1, s, 32, d)
    ks = lin(h, weights[1]).view(1, s, hkv, d)
    vs = lin(h, weights[2]).view(1, s, hkv, d) if family == "local" else ks
    q, _ = _prepare_reference(qs, weights[-2], cos, sin)
    k, _ = _prepare_reference(ks, weights[-1], cos, sin)
    v = _prepare_reference(vs, weights[-1], cos, sin, value=True)
    return _oracle_attention_out(family, q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2),
                                 weights[-3])


@pytest.mark.parametrize("family,s", [("local", 200), ("global", 128)])
def test_whole_layer_operator_matches_transformers_and_the_oracle(family, s):
    from gemma4_fa4_amd import transformers_integration as ti

    ops = _ops()
    cfg, module, _ = _module(family)
    weights = _weights(family)
    h = _hidden(s, s)
    pos = torch.arange(s, device=DEV)[None]
    cos, sin = _rope(family, pos)
    fwd = ops.local_layer_fwd if family == "local" else ops.global_layer_fwd
    with torch.inference_mode():
        out, lse = fwd(h, cos, sin, pos, torch.zeros_like(pos), *weights)
        ti.register_gemma4_mi355x()
        cfg._attn_implementation = ti.BACKEND_NAME
        hf_out, _ = module(h, (cos, sin), None, {})
    torch.cuda.synchronize()
    assert out.shape == (1, s, 5376) and lse.shape == (1, 32, s)
    fro_hf = rel_frobenius(out.float().cpu(), hf_out.float().cpu())
    assert fro_hf < 3e-3, f"vs Transformers with this backend: rel-Frobenius {fro_hf:.2e}"
    ref_out, ref_lse = _layer_reference(family, h, cos, sin, weights)
    fro = rel_frobenius(out.double().cpu(), ref_out)
    atol = LOCAL_LSE_ATOL if family == "local" else GLOBAL_LSE_ATOL
    lse_err = (lse.double().cpu() - ref_lse.double()).abs().max().item()
    print(f"{family} layer S={s}: rel-Fro vs HF {fro_hf:.2e}, vs fp64 {fro:.2e}, "
          f"LSE err {lse_err:.2e}")
    assert fro < 1e-2 and lse_err < atol


@pytest.mark.parametrize("family", ["local", "global"])
def test_compiled_layer_facade_equals_the_operator(family):
    import gemma4_fa4_amd as g4

    ops = _ops()
    weights = _weights(family)
    facade = g4.compile_gemma4_mi355x_layer(_module(family)[1])
    for s in (64, 65):  # dynamic shapes: one compiled frame
        h = _hidden(100 + s, s)
        pos = torch.arange(s, device=DEV)[None]
        cos, sin = _rope(family, pos)
        with torch.inference_mode():
            out, none = facade(h, (cos, sin), position_ids=pos)
            fwd = ops.local_layer_fwd if family == "local" else ops.global_layer_fwd
            ref, _ = fwd(h, cos, sin, pos, torch.zeros_like(pos), *weights)
        assert none is None and torch.equal(out, ref)
    assert facade.compiled_entry_count == 2


@pytest.mark.parametrize("family", ["local", "global"])
def test_whole_layer_opcheck_and_dormant_weight_flags(family):
    from gemma4_fa4_amd.errors import UnsupportedMI355XPath

    ops = _ops()
    weights = [w.detach().clone() for w in _weights(family)]
    s = 1
    pos = torch.arange(s, device=DEV)[None]
    cos, sin = _rope(family, pos)
    inputs = (_hidden(7, s), cos, sin, pos, torch.zeros_like(pos), *weights)
    op = ops.local_layer_op if family == "local" else ops.global_layer_op
    with torch.inference_mode():
        result = torch.library.opcheck(op, inputs)
    assert set(result.values()) == {"SUCCESS"}
    for w in weights:
        w.requires_grad_(True)
    fwd = ops.local_layer_fwd if family == "local" else ops.global_layer_fwd
    with torch.inference_mode():
        out, lse = fwd(*inputs[:5], *weights)
    assert not out.requires_grad and not lse.requires_grad
    with pytest.raises(UnsupportedMI355XPath, match="inference|no-grad"):
        fwd(*inputs[:5], *weights)


# --------------------------------------------------------------------------
# StaticCache decode
# --------------------------------------------------------------------------


def _filled_cache(family, capacity, length, seed):
    """K / V backings whose first `length` slots hold prepared rows of random sources."""
    f = FAMILY[family]
    g = torch.Generator().manual_seed(seed)
    shape = (1, f["hkv"], capacity, f["d"])
    sd = f["d"] ** -0.25
    k = torch.zeros(shape, dtype=torch.bfloat16)
    v = torch.zeros(shape, dtype=torch.bfloat16)
    k[:, :, :length] = (torch.randn(1, f["hkv"], length, f["d"], generator=g) * sd).bfloat16()
    v[:, :, :length] = torch.randn(1, f["hkv"], length, f["d"], generator=g).bfloat16()
    return k.to(DEV), v.to(DEV)


def _decode_reference(family, h, cos, sin, weights, cache_k, cache_v, active):
    """Expected new K / V rows and the fp64 output over the updated cache's first `active` slots."""
    f = FAMILY[family]
    lin = torch.nn.functional.linear
    d, hkv = f["d"], f["hkv"]
    qs = lin(h, weights[0]).view(1, 1, 32, d)
    ks = lin(h, weights[1]).view(1, 1, hkv, d)
    vs = lin(h, weights[2]).view(1, 1, hkv, d) if family == "local" else ks
    q, _ = _prepare_reference(qs, weights[-2], cos, sin)
    k_new, mag = _prepare_reference(ks, weights[-1], cos, sin)
    v_new = _prepare_reference(vs, weights[-1], cos, sin, value=True)
    return q, k_new, mag, v_new


def _check_decode_output(family, out, lse, q, cache_k, cache_v, active, o_weight):
    k = cache_k[:, :, :active].transpose(1, 2).cpu()
    v = cache_v[:, :, :active].transpose(1, 2).cpu()
    ref_out, ref_lse = _oracle_attention_out(family, q.transpose(1, 2), k, v, o_weight)
    fro = rel_frobenius(out.double().cpu(), ref_out)
    lse_err = (lse.double().cpu() - ref_lse.double()).abs().max().item()
    atol = LOCAL_LSE_ATOL if family == "local" else GLOBAL_LSE_ATOL
    assert fro < 1e-2 and lse_err < atol, f"{family} decode: fro {fro:.2e} lse {lse_err:.2e}"
    return fro


def test_global_decode_writes_the_next_slot_and_attends_the_prefix():
    ops = _ops()
    weights = _weights("global")
    length, capacity = 70, 100
    cache_k, cache_v = _filled_cache("global", capacity, length, 5)
    before_k, before_v = cache_k.clone(), cache_v.clone()
    cache_len = torch.tensor(length, device=DEV)
    pos = torch.tensor([[length]], device=DEV)
    cos, sin = _rope("global", pos)
    h = _hidden(9, 1)
    with torch.inference_mode():
        out, lse = ops.global_static_cache_decode_fwd(h, cos, sin, pos, cache_k, cache_v,
                                                      cache_len, *weights)
    torch.cuda.synchronize()
    assert int(cache_len) == length + 1 and out.shape == (1, 1, 5376) and lse.shape == (1, 32, 1)
    keep = torch.ones(capacity, dtype=torch.bool)
    keep[length] = False
    assert torch.equal(cache_k[:, :, keep], before_k[:, :, keep])
    assert torch.equal(cache_v[:, :, keep], before_v[:, :, keep])
    q, k_new, mag, v_new = _decode_reference("global", h, cos, sin, weights, cache_k, cache_v,
                                             length + 1)
    _ulp_check(cache_k[:, :, length:length + 1], k_new, "cache K", mag=mag, min_equal=0.99)
    _ulp_check(cache_v[:, :, length:length + 1], v_new, "cache V", min_equal=0.99)
    _check_decode_output("global", out, lse, q, cache_k, cache_v, length + 1, weights[-3])


@pytest.mark.parametrize("position", [100, 1500])
def test_local_decode_appends_or_rolls_the_window(position):
    ops = _ops()
    weights = _weights("local")
    stored = min(position, 1024)
    cache_k, cache_v = _filled_cache("local", 1024, stored, 6)
    before_k, before_v = cache_k.clone(), cache_v.clone()
    cache_len = torch.tensor(stored, device=DEV)
    pos = torch.tensor([[position]], device=DEV)
    cos, sin = _rope("local", pos)
    h = _hidden(10, 1)
    with torch.inference_mode():
        out, lse = ops.local_static_cache_decode_fwd(h, cos, sin, pos, cache_k, cache_v,
                                                     cache_len, *weights)
    torch.cuda.synchronize()
    assert int(cache_len) == stored  # the operator leaves the length to its caller
    if position < 1024:
        slot, active = position, position + 1
        keep = torch.ones(1024, dtype=torch.bool)
        keep[slot] = False
        assert torch.equal(cache_k[:, :, keep], before_k[:, :, keep])
        assert torch.equal(cache_v[:, :, keep], before_v[:, :, keep])
    else:
        slot, active = 1023, 1024
        assert torch.equal(cache_k[:, :, :1023], before_k[:, :, 1:])
        assert torch.equal(cache_v[:, :, :1023], before_v[:, :, 1:])
    q, k_new, mag, v_new = _decode_reference("local", h, cos, sin, weights, cache_k, cache_v,
                                             active)
    _ulp_check(cache_k[:, :, slot:slot + 1], k_new, "cache K", mag=mag, min_equal=0.99)
    _ulp_check(cache_v[:, :, slot:slot + 1], v_new, "cache V", min_equal=0.99)
    _check_decode_output("local", out, lse, q, cache_k, cache_v, active, weights[-3])


def test_decode_rejects_inconsistent_cache_state():
    from gemma4_fa4_amd.errors import UnsupportedMI355XPath

    ops = _ops()
    wg, wl = _weights("global"), _weights("local")
    h = _hidden(1, 1)
    ck, cv = _filled_cache("global", 72, 70, 1)
    cos, sin = _rope("global", torch.tensor([[70]]))
    with torch.inference_mode():
        with pytest.raises(UnsupportedMI355XPath, match="equal the active prefix"):
            ops.global_static_cache_decode_fwd(h, cos, sin, torch.tensor([[69]], device=DEV), ck,
                                               cv, torch.tensor(70, device=DEV), *wg)
        with pytest.raises(UnsupportedMI355XPath, match="spare"):
            ops.global_static_cache_decode_fwd(h, cos, sin, torch.tensor([[71]], device=DEV), ck,
                                               cv, torch.tensor(71, device=DEV), *wg)
        lk, lv = _filled_cache("local", 1024, 10, 2)
        cl, sl = _rope("local", torch.tensor([[10]]))
        with pytest.raises(UnsupportedMI355XPath, match="conflicts"):
            ops.local_static_cache_decode_fwd(h, cl, sl, torch.tensor([[10]], device=DEV), lk, lv,
                                              torch.tensor(9, device=DEV), *wl)


def _static_cache(cfg, capacity):
    cache = cache_utils.StaticCache(config=cfg, max_cache_len=capacity)
    cache.early_initialization(
        1, [16 if t == "sliding_attention" else 4 for t in cfg.layer_types],
        [256 if t == "sliding_attention" else 512 for t in cfg.layer_types],
        torch.bfloat16, torch.device(DEV))
    return cache


@pytest.mark.parametrize("family", ["local", "global"])
def test_decode_facade_steps_match_the_operator_and_keep_the_counters(family):
    import gemma4_fa4_amd as g4

    ops = _ops()
    cfg, module, _ = _module(family)
    weights = _weights(family)
    cache = _static_cache(cfg, 1100)
    layer = cache.layers[FAMILY[family]["layer"]]
    start = 1022 if family == "local" else 60
    fill_k, fill_v = _filled_cache(family, layer.keys.shape[2], min(start, 1024), 3)
    layer.keys.copy_(fill_k)
    layer.values.copy_(fill_v)
    layer.cumulative_length.fill_(min(start, 1024))
    if family == "local":
        layer.cumulative_length_int = start
    facade = g4.compile_gemma4_mi355x_static_cache_decode(module, cache)
    twin_k, twin_v = layer.keys.clone(), layer.values.clone()
    twin_len = layer.cumulative_length.clone()
    decode = ops.local_static_cache_decode_fwd if family == "local" else \
        ops.global_static_cache_decode_fwd
    for step in range(3):  # the local steps cross the window's capacity
        position = start + step
        pos = torch.tensor([[position]], device=DEV)
        cos, sin = _rope(family, pos)
        h = _hidden(50 + step, 1)
        with torch.inference_mode():
            out, none = facade(h, (cos, sin), position_ids=pos)
            ref, ref_lse = decode(h, cos, sin, pos, twin_k, twin_v, twin_len, *weights)
            if family == "local" and position < 1024:
                twin_len.add_(1)
        torch.cuda.synchronize()
        assert none is None and torch.equal(out, ref) and torch.equal(facade.last_lse, ref_lse)
        assert torch.equal(layer.keys, twin_k) and torch.equal(layer.values, twin_v)
        assert int(layer.cumulative_length) == int(twin_len)
        if family == "local":
            assert layer.cumulative_length_int == position + 1
            assert int(layer.cumulative_length) == min(position + 1, 1024)
        else:
            assert int(layer.cumulative_length) == position + 1
    assert facade.compiled_entry_count == 3
