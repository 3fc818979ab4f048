"""CPU tests of the drop-in boundary: library exports, validation, error classes.

Mirrors the reference's fake-backend adapter tests (tests/test_h100_fa4.py:43-1300):
every malformed input is rejected before any launch, with the reference's
exception types and messages.
"""

import subprocess
from dataclasses import replace

import pytest
import torch

import gemma4_fa4_amd as g
from gemma4_fa4_amd import _lib
from gemma4_fa4_amd import attention as att


def test_library_exports_every_declared_symbol():
    import os
    import re
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    header = open(os.path.join(root, "include", "gemma4_attn.h")).read()
    declared = set(re.findall(r"^\w[\w\s\*]*?\b(g4_\w+)\(", header, flags=re.M))
    assert declared == set(_lib.EXPORTED_SYMBOLS)
    lib = _lib.load()
    assert lib.g4_abi_version() == _lib.ABI_VERSION
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    for name in declared:
        assert re.search(rf"\bT {name}$", out, flags=re.M), name


def test_workspace_query_and_invalid_problem_are_reported():
    import ctypes
    lib = _lib.load()
    p = _lib.G4Problem(num_seqs=1, seqlen_q=128, seqlen_k=128, num_q_heads=32, num_kv_heads=16,
                       head_dim=256, window=1024)
    assert lib.g4_workspace_bytes(ctypes.byref(p), 0) == 0  # no vision: no span table
    assert lib.g4_workspace_bytes(ctypes.byref(p), 1) >= 32 * 128 * 4
    bad = _lib.G4Problem(num_seqs=1, seqlen_q=128, seqlen_k=128, num_q_heads=32,
                         num_kv_heads=16, head_dim=128)
    assert lib.g4_workspace_bytes(ctypes.byref(bad), 0) == 0
    assert b"head_dim" in lib.g4_last_error()
    with pytest.raises(g.UnsupportedMI355XPath, match="head_dim"):
        _lib.check(_lib.G4_ERR_UNSUPPORTED)


def test_an_earlier_rejection_does_not_fail_a_later_valid_problem():
    # g4_last_error is per call: a rejected problem on this thread must not make
    # a later valid problem whose workspace is legitimately 0 bytes look failed.
    import ctypes
    lib = _lib.load()
    bad = _lib.G4Problem(num_seqs=1, seqlen_q=128, seqlen_k=128, num_q_heads=32,
                         num_kv_heads=16, head_dim=128)
    assert lib.g4_workspace_bytes(ctypes.byref(bad), 0) == 0
    assert lib.g4_last_error()
    good = _lib.G4Problem(num_seqs=1, seqlen_q=128, seqlen_k=128, num_q_heads=32,
                          num_kv_heads=16, head_dim=256, window=1024)
    assert lib.g4_workspace_bytes(ctypes.byref(good), 0) == 0
    assert lib.g4_last_error() == b""
    plan = att._Plan(packed=False, num_seqs=1, seqlen_q=128, seqlen_k=128, num_q_heads=32,
                     num_kv_heads=16, head_dim=256, window=1024, bidirectional=False,
                     total_q=128, total_k=128)
    lib.g4_workspace_bytes(ctypes.byref(bad), 1)
    assert plan.workspace_bytes(0) == 0  # does not raise


def _ws(**kw):
    import ctypes
    p = _lib.G4Problem(num_seqs=1, num_q_heads=32, **kw)
    return _lib.load().g4_workspace_bytes(ctypes.byref(p), 1)


def test_ds_budget_sizes_the_stored_dS_tiles():
    # head dim 512 causal, S=4096: 128 rows x 64 key tiles x 32 heads x 4 KB
    d512 = dict(seqlen_q=4096, seqlen_k=4096, num_kv_heads=4, head_dim=512, window=0)
    dense = 128 * 64 * 32 * 4096
    assert _ws(**d512) - _ws(**d512, ds_budget=-1) == dense
    assert _ws(**d512, ds_budget=dense) - _ws(**d512, ds_budget=-1) == dense
    # Past the budget the one sequence is striped: fp32 dK / dV sums (2 x 4096
    # keys x 4 KV heads x 512 x 4 B) plus the largest stripe must fit it.  With
    # room for 2048 (row, key tile) units of 32 x 4 KB after the sums, rows
    # [0, 64) reach 32 key tiles (64 x 32 = 2048 units), rows [64, 100) reach
    # 50 (1800; 40 rows would need 40 x 52 = 2080), rows [100, 128) all 64 (1792).
    sums = 2 * 4096 * 4 * 512 * 4
    unit = 32 * 4096
    budget = sums + 2048 * unit
    assert _ws(**d512, ds_budget=budget) - _ws(**d512, ds_budget=-1) == sums + 2048 * unit
    # one byte less: rows [0, 60) x 30 key tiles (1800), rows [60, 100) x 50
    # (2000; 44 rows would need 44 x 52), rows [100, 128) x 64 (1792)
    assert _ws(**d512, ds_budget=budget - 1) - _ws(**d512, ds_budget=-1) == sums + 2000 * unit
    # the last four rows reach all 64 key tiles: below 4 x 64 units after the
    # sums nothing is stored (the dQ stage recomputes); at it, stripes of at
    # most 256 units
    assert _ws(**d512, ds_budget=sums + 4 * 64 * unit - 1) == _ws(**d512, ds_budget=-1)
    assert _ws(**d512, ds_budget=sums + 4 * 64 * unit) - _ws(**d512, ds_budget=-1) == (
        sums + 256 * unit)
    # head dim 256 window 1024: a band of (1024 + 30) // 64 + 2 = 18 key tiles per row
    d256 = dict(seqlen_q=4096, seqlen_k=4096, num_kv_heads=16, head_dim=256, window=1024)
    band = 128 * 18 * 32 * 4096
    assert _ws(**d256) - _ws(**d256, ds_budget=-1) == band
    assert _ws(**d256, ds_budget=band - 1) == _ws(**d256, ds_budget=-1)
    # the default budget is 16 GiB: exactly a 16384-token global sequence's tiles;
    # one more 32-query row and the sequence is striped within the 16 GiB
    at = dict(seqlen_q=16384, seqlen_k=16384, num_kv_heads=4, head_dim=512, window=0)
    assert _ws(**at) - _ws(**at, ds_budget=-1) == 16 << 30
    big = dict(seqlen_q=16416, seqlen_k=16416, num_kv_heads=4, head_dim=512, window=0)
    striped = _ws(**big) - _ws(**big, ds_budget=-1)
    big_sums = 2 * 16416 * 4 * 512 * 4
    assert big_sums < striped <= 16 << 30 and (striped - big_sums) % unit == 0
    assert _ws(**big, ds_budget=1 << 36) - _ws(**big, ds_budget=-1) == 513 * 257 * 32 * 4096
    # a packed batch is never striped: past the budget its dQ stage recomputes
    two = dict(num_kv_heads=4, head_dim=512, window=0)
    p2 = _lib.G4Problem(num_seqs=2, num_q_heads=32, seqlen_q=4096, seqlen_k=4096, **two)
    import ctypes
    lib = _lib.load()
    p2.ds_budget = -1
    lean = lib.g4_workspace_bytes(ctypes.byref(p2), 1)
    p2.ds_budget = budget
    assert lib.g4_workspace_bytes(ctypes.byref(p2), 1) == lean


def test_ds_budget_sequence_stripes_of_several_sequences():
    # Several d512 causal sequences past the budget are striped by sequence:
    # stripe k takes the sequences whose first dS row lies in [k H, (k + 1) H)
    # and needs H + 63 buffer rows (the longest sequence, 2048 queries, has 64
    # rows), with H as large as fits and at least 64; no fp32 sums.
    import ctypes
    lib = _lib.load()
    cu = (ctypes.c_int32 * 5)(0, 1000, 3048, 3100, 4096)  # never read on the host
    per_row = 32 * 32 * 4096  # 32 key tiles x 32 heads x 4 KB

    def ws(budget, packed=True):
        p = _lib.G4Problem(num_seqs=4, seqlen_q=2048, seqlen_k=2048, num_q_heads=32,
                           num_kv_heads=4, head_dim=512, window=0, total_q=4096,
                           total_k=4096, ds_budget=budget)
        if packed:
            p.cu_seqlens_q = p.cu_seqlens_k = ctypes.cast(cu, ctypes.c_void_p)
        return lib.g4_workspace_bytes(ctypes.byref(p), 1)

    lean = ws(-1)
    assert ws(0) - lean == (4096 // 32 + 4) * per_row  # dense: 132 packed rows fit 16 GiB
    assert ws(132 * per_row) - lean == 132 * per_row
    # 127 rows: H = 127 - 63 = 64, stripes from rows 0, 64, 128 (127, 68 and 4 rows)
    assert ws(127 * per_row) - lean == 127 * per_row
    assert ws(131 * per_row) - lean == 131 * per_row  # H = 68: stripes of 131 and 64 rows
    # 126 rows: H = 63 < 64, recompute
    assert ws(127 * per_row - 1) == lean
    # fixed layout, 4 x 2048: 256 rows; 200 rows give H = 137 (stripes of 200, 119)
    flean = ws(-1, packed=False)
    assert ws(200 * per_row, packed=False) - flean == 200 * per_row
    assert ws(0, packed=False) - flean == 256 * per_row


@pytest.mark.parametrize("make,ok", [
    (lambda: torch.zeros(1, 64, 32, 256, dtype=torch.bfloat16), True),
    (lambda: torch.zeros(256, dtype=torch.bfloat16).expand(1, 64, 32, 256), False),
    (lambda: torch.zeros(64, 32, 264, dtype=torch.bfloat16)[..., :256], True),
    (lambda: torch.zeros(64 * 32 * 256 + 8, dtype=torch.bfloat16)[1:64 * 32 * 256 + 1]
     .view(64, 32, 256), False),  # base off 16-byte alignment
    (lambda: torch.zeros(64, 32, 260, dtype=torch.bfloat16)[..., :256], False),
])
def test_upstream_gradient_operand_contract(make, ok):
    # The backward copies an upstream gradient the library would reject
    # (broadcast, misaligned) instead of failing a valid autograd graph.
    assert att._meets_operand_contract(make()) is ok


def test_error_hierarchy_keeps_reference_names():
    assert issubclass(g.GlobalBackwardBudgetExceeded, g.UnsupportedH100Path)
    assert g.UnsupportedH100Path is g.UnsupportedMI355XPath
    assert issubclass(g.UnsupportedMI355XPath, RuntimeError)


def _local(seqlen=2):
    s = g.SLIDING_ATTENTION
    q = torch.zeros(1, seqlen, s.num_q_heads, s.head_dim_qk, dtype=torch.bfloat16)
    k = torch.ones(1, seqlen, s.num_kv_heads, s.head_dim_qk, dtype=torch.bfloat16)
    v = torch.full((1, seqlen, s.num_kv_heads, s.head_dim_v), 2, dtype=torch.bfloat16)
    return q, k, v


def test_valid_cpu_inputs_fail_only_on_the_device_check():
    with pytest.raises(g.UnsupportedMI355XPath, match="GPU tensors"):
        g.fa4_local_text_forward(*_local())


@pytest.mark.parametrize("mutate,exc,match", [
    (lambda q, k, v: (q.float(), k, v), ValueError, "BF16"),
    (lambda q, k, v: (q[..., :128], k, v), ValueError, "shape"),
    (lambda q, k, v: (q, k, k), ValueError, "distinct"),
    (lambda q, k, v: (q.transpose(-1, -2).contiguous().transpose(-1, -2), k, v), ValueError,
     "unit last"),
    (lambda q, k, v: (q[0], k[0], v[0]), ValueError, "rank-4"),
])
def test_local_fixed_rejects_malformed_inputs(mutate, exc, match):
    with pytest.raises(exc, match=match):
        g.fa4_local_text_forward(*mutate(*_local()))


def test_local_fixed_envelope_is_b1_s1025(monkeypatch):
    monkeypatch.setattr(att, "_require_gfx950", lambda _device: None)
    with pytest.raises(g.UnsupportedMI355XPath, match="S <= 1025"):
        g.fa4_local_text_forward(*_local(1026))
    q, k, v = _local()
    with pytest.raises(g.UnsupportedMI355XPath, match="B=1"):
        g.fa4_local_text_forward(q.expand(2, -1, -1, -1).contiguous(),
                                 k.expand(2, -1, -1, -1).contiguous(),
                                 v.expand(2, -1, -1, -1).contiguous())


def test_local_spec_must_be_the_locked_contract(monkeypatch):
    monkeypatch.setattr(att, "_require_gfx950", lambda _device: None)
    with pytest.raises(g.UnsupportedMI355XPath, match="locked local"):
        g.fa4_local_text_forward(*_local(), spec=replace(g.SLIDING_ATTENTION, softmax_scale=0.5))


def test_vision_ids_are_validated_and_normalised(monkeypatch):
    monkeypatch.setattr(att, "_require_gfx950", lambda _device: None)
    q, k, v = _local(4)
    with pytest.raises(ValueError, match="shape"):
        g.fa4_local_forward(q, k, v, vision_block_ids=torch.zeros(1, 3, dtype=torch.int32))
    with pytest.raises(ValueError, match="INT32 or INT64"):
        g.fa4_local_forward(q, k, v, vision_block_ids=torch.zeros(1, 4))
    with pytest.raises(ValueError, match="fit exactly in INT32"):
        att._normalize_int32_metadata(torch.tensor([2**40]), name="vision_block_ids")
    ids = att._prepare_vision_block_ids(torch.tensor([[-1, 0, 0, -1]]), q)
    assert ids.dtype == torch.int32 and ids.shape == (4,) and ids.is_contiguous()


def _packed(q_lengths=(2, 1), k_lengths=(3, 2)):
    s = g.SLIDING_ATTENTION
    q = torch.zeros(sum(q_lengths), s.num_q_heads, s.head_dim_qk, dtype=torch.bfloat16)
    k = torch.ones(sum(k_lengths), s.num_kv_heads, s.head_dim_qk, dtype=torch.bfloat16)
    v = torch.full_like(k, 2)
    cq = torch.tensor([0, *torch.tensor(q_lengths).cumsum(0).tolist()], dtype=torch.int32)
    ck = torch.tensor([0, *torch.tensor(k_lengths).cumsum(0).tolist()], dtype=torch.int32)
    return q, k, v, cq, ck


def test_local_varlen_validation():
    q, k, v, cq, ck = _packed()
    with pytest.raises(TypeError, match="Python integers"):
        g.fa4_local_varlen_forward(q, k, v, cq, ck, max_seqlen_q=2.0, max_seqlen_k=3)
    with pytest.raises(ValueError, match="INT32"):
        g.fa4_local_varlen_forward(q, k, v, cq.long(), ck.long(), max_seqlen_q=2, max_seqlen_k=3)
    with pytest.raises(ValueError, match="maxima"):
        g.fa4_local_varlen_forward(q, k, v, cq, ck, max_seqlen_q=1, max_seqlen_k=3)
    with pytest.raises(g.UnsupportedMI355XPath, match="Sq <= Sk"):
        g.fa4_local_varlen_forward(*_packed((3, 1), (2, 4)), max_seqlen_q=3, max_seqlen_k=4)
    bad = torch.tensor([0, 2, 1], dtype=torch.int32)
    with pytest.raises(ValueError, match="end at|nondecreasing"):
        g.fa4_local_varlen_forward(q, k, v, bad, ck, max_seqlen_q=2, max_seqlen_k=3)
    with pytest.raises(g.UnsupportedMI355XPath, match="GPU tensors"):
        g.fa4_local_varlen_forward(q, k, v, cq, ck, max_seqlen_q=2, max_seqlen_k=3)
    with pytest.raises(g.UnsupportedMI355XPath, match="262144"):
        g.fa4_local_varlen_forward(q, k, v, cq, ck, max_seqlen_q=2, max_seqlen_k=262145)


def test_global_adapters_validation(monkeypatch):
    monkeypatch.setattr(att, "_require_gfx950", lambda _device: None)
    s = g.GLOBAL_ATTENTION
    q = torch.zeros(1, 2049, 32, 512, dtype=torch.bfloat16)
    k = torch.zeros(1, 2049, 4, 512, dtype=torch.bfloat16)
    v = torch.zeros(1, 2049, 4, 512, dtype=torch.bfloat16)
    with pytest.raises(g.UnsupportedMI355XPath, match="S <= 2048"):
        g.fa4_global_text_forward(q, k, v)
    qg = q[:, :8].clone().requires_grad_(True)
    with pytest.raises(g.UnsupportedMI355XPath, match="autograd"):
        g.fa4_global_forward_only(qg, k[:, :8].clone(), v[:, :8].clone())
    with pytest.raises(g.UnsupportedMI355XPath, match="locked global"):
        g.fa4_global_forward_only(q[:, :8], k[:, :8], v[:, :8],
                                  spec=replace(s, sliding_window=1024))


def test_global_backward_budget_fails_closed():
    free = 10 * 1024**3
    budget = att._global_backward_budget(free)
    assert budget == min(free * 4 // 5, free - 2 * 1024**3)
    att._check_global_backward_budget(budget, free)
    with pytest.raises(g.GlobalBackwardBudgetExceeded):
        att._check_global_backward_budget(budget + 1, free)


def _global_packed(lengths=(3, 2)):
    s = g.GLOBAL_ATTENTION
    t = sum(lengths)
    q = torch.zeros(t, s.num_q_heads, 512, dtype=torch.bfloat16)
    k = torch.ones(t, s.num_kv_heads, 512, dtype=torch.bfloat16)
    v = torch.full_like(k, 2)
    cu = torch.tensor([0, *torch.tensor(lengths).cumsum(0).tolist()], dtype=torch.int32)
    return q, k, v, cu


def test_cumulative_arrays_are_read_at_launch(monkeypatch):
    """The cu_seqlens read (a stream sync) follows the preflight and the allocation."""
    monkeypatch.setattr(att, "_require_gfx950", lambda _device: None)
    calls = []
    real = att._cumulative_lengths
    monkeypatch.setattr(att, "_cumulative_lengths",
                        lambda *a, **kw: (calls.append("read"), real(*a, **kw))[1])
    monkeypatch.setattr(att, "_preflight_forward_outputs", lambda _q: calls.append("preflight"))

    def no_library():
        calls.append("load")
        raise g.UnsupportedMI355XPath("library withheld by the test")

    monkeypatch.setattr(_lib, "load", no_library)
    q, k, v, cu = _global_packed()
    with pytest.raises(g.UnsupportedMI355XPath, match="withheld"):
        g.fa4_global_varlen_forward_only(q, k, v, cu, cu, max_seqlen_q=3, max_seqlen_k=3)
    assert calls == ["preflight", "load", "read"]
    # Invalid arrays still report their own error before the later failure.
    calls.clear()
    with pytest.raises(ValueError, match="maxima"):
        g.fa4_global_varlen_forward_only(q, k, v, cu, cu, max_seqlen_q=4, max_seqlen_k=4)
    assert calls == ["preflight", "load", "read"]


def test_held_errors_follow_the_length_checks(monkeypatch):
    monkeypatch.setattr(att, "_require_gfx950", lambda _device: None)

    def refuse(_q):
        raise g.UnsupportedMI355XPath("preflight refused by the test")

    monkeypatch.setattr(att, "_preflight_forward_outputs", refuse)
    q, k, v, cu = _global_packed()
    bad = torch.tensor([0, 4, 5], dtype=torch.int32)
    with pytest.raises(ValueError, match="maxima"):
        g.fa4_global_varlen_forward_only(q, k, v, bad, bad, max_seqlen_q=3, max_seqlen_k=3)
    with pytest.raises(g.UnsupportedMI355XPath, match="refused by the test"):
        g.fa4_global_varlen_forward_only(q, k, v, cu, cu, max_seqlen_q=3, max_seqlen_k=3)


def test_model_contract_constants():
    s, f = g.SLIDING_ATTENTION, g.GLOBAL_ATTENTION
    assert (s.head_dim_qk, s.num_q_heads, s.num_kv_heads, s.sliding_window) == (256, 32, 16, 1024)
    assert s.fa_window_size_left == 1023 and s.softmax_scale == 1.0
    assert (f.head_dim_qk, f.num_q_heads, f.num_kv_heads, f.sliding_window) == (512, 32, 4, None)
    types = g.GEMMA4_31B.layer_types()
    assert len(types) == 60 and types.count("full_attention") == 10
    assert types[5] == "full_attention" and types[4] == "sliding_attention"
    assert f.rotary_dim == 128 and f.qhead_per_kvhead == 8 and s.qhead_per_kvhead == 2


def test_cumulative_host_copies_are_reused_only_while_unchanged(monkeypatch):
    cache = att._HostValues(capacity=2)
    monkeypatch.setattr(att, "_CU_HOST", cache)
    copies = []
    real_cpu = torch.Tensor.cpu

    def counting_cpu(self, *a, **kw):
        copies.append(1)
        return real_cpu(self, *a, **kw)

    monkeypatch.setattr(torch.Tensor, "cpu", counting_cpu)
    cu = torch.tensor([0, 5, 9], dtype=torch.int32)
    assert att._host_values(cu, cu) == ([0, 5, 9], [0, 5, 9]) and len(copies) == 1
    assert att._host_values(cu, cu) == ([0, 5, 9], [0, 5, 9]) and len(copies) == 1
    cu[1] = 4  # in-place change: read again
    assert att._host_values(cu, cu)[0] == [0, 4, 9] and len(copies) == 2
    cu.view(3)[2].add_(1)  # through a view
    assert att._host_values(cu, cu)[0] == [0, 4, 10] and len(copies) == 3
    other = cu.clone()  # equal values, different tensor: read
    assert att._host_values(other, other)[0] == [0, 4, 10] and len(copies) == 4
    cq, ck = torch.tensor([0, 3], dtype=torch.int32), torch.tensor([0, 7], dtype=torch.int32)
    assert att._host_values(cq, ck) == ([0, 3], [0, 7]) and len(copies) == 5
    assert att._host_values(cq, ck) == ([0, 3], [0, 7]) and len(copies) == 5
    with torch.inference_mode():
        inf = torch.tensor([0, 2], dtype=torch.int32)
    att._host_values(inf, inf)
    att._host_values(inf, inf)
    assert len(copies) == 7  # inference tensors are always read


def test_static_workspace_forward_rejects_a_problem_beyond_its_array():
    # Host-side check before any device call: vision span tables of 2^20 K
    # tokens need 40 MiB, more than the 32 MiB static forward workspace.
    import ctypes
    lib = _lib.load()
    t = 1 << 20
    p = _lib.G4Problem(num_seqs=1, seqlen_q=t, seqlen_k=t, num_q_heads=32, num_kv_heads=16,
                       head_dim=256, window=1024, bidirectional_vision=1, total_q=t, total_k=t,
                       cu_seqlens_q=0x1000, cu_seqlens_k=0x1000, vision_ids=0x2000,
                       lse_head_stride=t)
    assert lib.g4_workspace_bytes(ctypes.byref(p), 0) > _lib.STATIC_WORKSPACE_BYTES
    lay = _lib.G4Layout(0, 32 * 256, 256)
    kv = _lib.G4Layout(0, 16 * 256, 256)
    rc = lib.g4_attn_fwd_static(ctypes.byref(p), 0x10000, lay, 0x20000, kv, 0x30000, kv,
                                0x40000, lay, 0x50000, None)
    assert rc == _lib.G4_ERR_WORKSPACE
    assert b"static forward workspace" in lib.g4_last_error()


def test_backward_budget_drops_stored_ds_before_failing(monkeypatch):
    # The dS tiles are stored only while gradients + workspace fit the
    # reference's budget (80% of free HBM, at most free - 2 GiB); past it the
    # one sequence is striped within what is left, and below the fp32 sums plus
    # four rows of tiles the dQ stage recomputes (lean workspace); only when
    # even that does not fit is GlobalBackwardBudgetExceeded raised
    # (h100.py:713-746 policy).
    s = 4096
    q = torch.empty(s, 32, 512, dtype=torch.bfloat16)
    k = torch.empty(s, 4, 512, dtype=torch.bfloat16)
    v = torch.empty(s, 4, 512, dtype=torch.bfloat16)
    cu = torch.tensor([0, s], dtype=torch.int32)
    plan = att._packed_plan(q, k, cu, cu, s, s, g.GLOBAL_ATTENTION)
    plan.ds_budget = 0
    full = att._backward_additional_bytes(plan, q, k, v)
    plan.ds_budget = -1
    lean = att._backward_additional_bytes(plan, q, k, v)
    assert full - lean == (s // 32 + 1) * 64 * 32 * 4096  # the stored dS tiles (packed rows)
    gib = 1024 ** 3

    def free_for(budget):  # free bytes whose budget is `budget`
        return max(budget * 5 // 4 + 4, budget + 2 * gib)

    monkeypatch.setattr(att, "_free_hbm", lambda _d: free_for(full))
    att._preflight_backward(plan, q, k, v)
    assert plan.ds_budget == 0  # everything fits: default budget, tiles stored
    monkeypatch.setattr(att, "_free_hbm", lambda _d: free_for(full - 1))
    att._preflight_backward(plan, q, k, v)
    assert plan.ds_budget > 0 and lean < att._backward_additional_bytes(plan, q, k, v) < full
    sums, last_rows = 2 * s * 4 * 512 * 4, 4 * 64 * 32 * 4096
    monkeypatch.setattr(att, "_free_hbm", lambda _d: free_for(lean + sums + last_rows))
    att._preflight_backward(plan, q, k, v)
    assert att._backward_additional_bytes(plan, q, k, v) == lean + sums + last_rows
    monkeypatch.setattr(att, "_free_hbm", lambda _d: free_for(lean + sums + last_rows - 1))
    att._preflight_backward(plan, q, k, v)
    assert plan.ds_budget > 0 and att._backward_additional_bytes(plan, q, k, v) == lean
    monkeypatch.setattr(att, "_free_hbm", lambda _d: free_for(lean - 1))
    with pytest.raises(g.GlobalBackwardBudgetExceeded):
        att._preflight_backward(plan, q, k, v)


def _global_plan_s4096():
    s = 4096
    q = torch.empty(s, 32, 512, dtype=torch.bfloat16)
    k = torch.empty(s, 4, 512, dtype=torch.bfloat16)
    v = torch.empty(s, 4, 512, dtype=torch.bfloat16)
    cu = torch.tensor([0, s], dtype=torch.int32)
    return att._packed_plan(q, k, cu, cu, s, s, g.GLOBAL_ATTENTION), q, k, v


def _free_for(budget):  # free bytes whose guarded budget is `budget`
    return max(budget * 5 // 4 + 4, budget + 2 * 1024 ** 3)


def test_backward_refits_the_ds_budget_when_free_hbm_shrinks(monkeypatch):
    # The forward fits the stored-dS route to the HBM free then; by the
    # backward other allocations may have taken it.  The backward fits again
    # before allocating (patch 0002:1164-1181 measures free HBM there): the
    # recompute route when the tiles no longer fit, the typed error when even
    # that does not.
    plan, q, k, v = _global_plan_s4096()
    plan.ds_budget = 0
    full = att._backward_additional_bytes(plan, q, k, v)
    plan.ds_budget = -1
    lean = att._backward_additional_bytes(plan, q, k, v)
    monkeypatch.setattr(att, "_free_hbm", lambda _d: _free_for(full))
    att._preflight_backward(plan, q, k, v)  # forward time: everything fits
    assert plan.ds_budget == 0 and plan.global_backward
    monkeypatch.setattr(att, "_free_hbm", lambda _d: _free_for(lean))
    att._refit_backward(plan, q, k, v)  # backward time: only the lean route fits
    assert att._backward_additional_bytes(plan, q, k, v) == lean
    monkeypatch.setattr(att, "_free_hbm", lambda _d: _free_for(full))
    att._refit_backward(plan, q, k, v)  # memory came back: tiles stored again
    assert plan.ds_budget == 0
    monkeypatch.setattr(att, "_free_hbm", lambda _d: _free_for(lean - 1))
    with pytest.raises(g.GlobalBackwardBudgetExceeded):
        att._refit_backward(plan, q, k, v)
    # a local layer shrinks its band instead of failing
    local = att._packed_plan(q[:, :, :256], k[:, :, :256].repeat(1, 4, 1), plan.cu_q, plan.cu_k,
                             4096, 4096, g.SLIDING_ATTENTION)
    monkeypatch.setattr(att, "_free_hbm", lambda _d: 1)
    att._refit_backward(local, q[:, :, :256], k[:, :, :256].repeat(1, 4, 1),
                        v[:, :, :256].repeat(1, 4, 1))
    assert local.ds_budget < 0 and not local.global_backward


def test_backward_fits_before_it_allocates(monkeypatch):
    plan, q, k, v = _global_plan_s4096()

    class Refit(Exception):
        pass

    def refit(*_a):
        raise Refit

    monkeypatch.setattr(att, "_refit_backward", refit)
    allocated = []
    monkeypatch.setattr(plan, "_workspace", lambda *a, **kw: allocated.append(a))
    with pytest.raises(Refit):
        plan.backward(q, k, v, q, q, torch.empty(32, 4096), None)
    assert not allocated


def test_pinned_ds_budget_fixes_the_route(monkeypatch):
    # With the budget pinned the route no longer depends on the free HBM (the
    # two routes sum dQ in different orders); the global layer still fails
    # closed when the pinned route does not fit.
    plan, q, k, v = _global_plan_s4096()
    plan.ds_budget = -1
    lean = att._backward_additional_bytes(plan, q, k, v)
    monkeypatch.setattr(att, "_free_hbm", lambda _d: 1 << 50)
    previous = g.pin_backward_ds_budget(-1)
    try:
        assert previous is None
        att._preflight_backward(plan, q, k, v)
        assert plan.ds_budget == -1
        att._refit_backward(plan, q, k, v)
        assert plan.ds_budget == -1
        monkeypatch.setattr(att, "_free_hbm", lambda _d: _free_for(lean - 1))
        with pytest.raises(g.GlobalBackwardBudgetExceeded):
            att._refit_backward(plan, q, k, v)
        with pytest.raises(TypeError):
            g.pin_backward_ds_budget(1.5)
    finally:
        assert g.pin_backward_ds_budget(previous) == -1
    monkeypatch.setattr(att, "_free_hbm", lambda _d: 1 << 50)
    att._refit_backward(plan, q, k, v)
    assert plan.ds_budget == 0


def test_row_preparation_validation_happens_before_any_launch():
    # Host-side checks of g4_kv_prep_fwd / _bwd with fake addresses: nothing
    # reaches the device when a check fails.
    import ctypes
    lib = _lib.load()
    lay = _lib.G4Layout(0, 16 * 256, 256)
    p = _lib.G4KvPrep(num_batches=1, seqlen=4, num_heads=16, head_dim=256, rotary_dim=256,
                      k_fp32=0, eps=1e-6, cs_batch_stride=0)
    assert lib.g4_kv_prep_fwd(ctypes.byref(p), 0x1000, lay, 0x2000, 0x3000, 0x4000, None, lay,
                              None, lay, None) == _lib.G4_ERR_INVALID
    assert b"both K and V are NULL" in lib.g4_last_error()
    # a K output needs the rotary tables; a V-only call does not
    assert lib.g4_kv_prep_fwd(ctypes.byref(p), 0x1000, lay, 0x2000, None, None, 0x5000, lay,
                              None, lay, None) == _lib.G4_ERR_INVALID
    assert b"cos and sin" in lib.g4_last_error()
    assert lib.g4_kv_prep_fwd(ctypes.byref(p), 0x1000, lay, 0x2003, None, None, None, lay,
                              0x6000, lay, None) == _lib.G4_ERR_INVALID
    assert b"weight" in lib.g4_last_error()
    odd = _lib.G4KvPrep(num_batches=1, seqlen=4, num_heads=16, head_dim=384, rotary_dim=0,
                        k_fp32=0, eps=1e-6, cs_batch_stride=0)
    assert lib.g4_kv_prep_fwd(ctypes.byref(odd), 0x1000, lay, 0x2000, None, None, None, lay,
                              0x6000, lay, None) == _lib.G4_ERR_UNSUPPORTED
    # the backward covers head_dim 512 only
    assert lib.g4_kv_prep_bwd(ctypes.byref(p), 0x1000, lay, 0x2000, 0x3000, 0x4000, 0x5000, lay,
                              0x6000, lay, 0x7000, lay, 0x8000, 0x9000, 1 << 20,
                              None) == _lib.G4_ERR_UNSUPPORTED
    assert b"head_dim 512" in lib.g4_last_error()


def test_forward_checks_reuse_a_recent_free_hbm_reading(monkeypatch):
    """The forward-time checks reuse a hipMemGetInfo reading for 20 ms; a
    replaced ``_free_hbm`` is always consulted, and the backward's refit reads
    afresh through ``_free_hbm`` itself."""
    import time

    calls = []

    def mem_get_info(device):
        calls.append(device)
        return (1000 + len(calls), 2000)

    monkeypatch.setattr(torch.cuda, "mem_get_info", mem_get_info)
    monkeypatch.setattr(att, "_FREE_HBM_READINGS", {})
    dev = torch.device("cuda", 0)
    assert att._recent_free_hbm(dev) == 1001
    assert att._recent_free_hbm(dev) == 1001 and len(calls) == 1  # reused
    assert att._free_hbm(dev) == 1002  # always a fresh read (the backward's refit)
    assert att._recent_free_hbm(dev) == 1002 and len(calls) == 2
    monkeypatch.setattr(att, "_FREE_HBM_REUSE_S", 0.0)
    time.sleep(0.001)
    assert att._recent_free_hbm(dev) == 1003  # expired: read again
    monkeypatch.setattr(att, "_FREE_HBM_REUSE_S", 60.0)
    monkeypatch.setattr(att, "_free_hbm", lambda _d: 7)
    assert att._recent_free_hbm(dev) == 7  # a replaced reader is never bypassed
