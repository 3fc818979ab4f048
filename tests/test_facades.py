"""Host contract of the guarded compiled facades (CPU; real Transformers modules).

Builds the installed Transformers ``Gemma4TextAttention`` at the Gemma 4 31B
attention geometry (a sliding layer and a global layer) and checks what the
reference's facades check before any launch
(src/gemma4_fa4/transformers_integration.py:2144-2211, 2599-2736): the module
contract and its explicit weight tuple, StaticCache layer binding, and that a
call off the GPU fails explicitly.
"""

from __future__ import annotations

import pytest
import torch

import gemma4_fa4_amd as g
from gemma4_fa4_amd import facades
from gemma4_fa4_amd.errors import UnsupportedMI355XPath

mg = pytest.importorskip("transformers.models.gemma4.modeling_gemma4")
cu = pytest.importorskip("transformers.cache_utils")


def _config():
    from transformers.models.gemma4.configuration_gemma4 import Gemma4TextConfig

    return Gemma4TextConfig(hidden_size=5376, num_attention_heads=32, num_key_value_heads=16,
                            head_dim=256, global_head_dim=512, num_global_key_value_heads=4,
                            attention_k_eq_v=True, sliding_window=1024, num_hidden_layers=60,
                            hidden_size_per_layer_input=0, vocab_size_per_layer_input=0,
                            max_position_embeddings=262144)


@pytest.fixture(scope="module")
def modules():
    torch.manual_seed(0)
    cfg = _config()
    with torch.device("cpu"):
        local = mg.Gemma4TextAttention(cfg, 0).to(torch.bfloat16).eval()
        glob = mg.Gemma4TextAttention(cfg, 5).to(torch.bfloat16).eval()
    return cfg, local, glob


def test_layer_weights_follow_the_operator_argument_order(modules):
    _, local, glob = modules
    wl = facades.layer_weights(local)
    assert [w.shape for w in wl] == [(8192, 5376), (4096, 5376), (4096, 5376), (5376, 8192),
                                     (256,), (256,)]
    assert wl[0] is local.q_proj.weight and wl[2] is local.v_proj.weight
    wg = facades.layer_weights(glob)
    assert [w.shape for w in wg] == [(16384, 5376), (2048, 5376), (5376, 16384), (512,), (512,)]
    assert glob.v_proj is None and wg[3] is glob.q_norm.weight


def test_module_contract_fails_closed(modules):
    _, local, glob = modules
    local.train()
    try:
        with pytest.raises(UnsupportedMI355XPath, match="eval-mode"):
            facades.layer_weights(local)
    finally:
        local.eval()
    fp32 = local.q_proj.weight.data
    local.q_proj.weight.data = fp32.float()
    try:
        with pytest.raises(UnsupportedMI355XPath, match="q_proj"):
            facades.layer_weights(local)
    finally:
        local.q_proj.weight.data = fp32
    with pytest.raises(UnsupportedMI355XPath, match="Gemma4TextAttention"):
        facades.layer_weights(object.__new__(type("Fake", (), {"layer_idx": 0})))


def test_facades_build_and_refuse_off_gpu_calls(modules):
    cfg, local, glob = modules
    facade = g.compile_gemma4_mi355x_layer(glob)
    assert facade.compiled_entry_count == 0
    h = torch.zeros(1, 4, 5376, dtype=torch.bfloat16)
    rope = (torch.ones(1, 4, 512, dtype=torch.bfloat16), torch.zeros(1, 4, 512, dtype=torch.bfloat16))
    with torch.no_grad(), pytest.raises(UnsupportedMI355XPath, match="CUDA"):
        facade(h, rope, position_ids=torch.arange(4)[None])
    with pytest.raises(UnsupportedMI355XPath, match="no-grad"):
        facade(h, rope, position_ids=torch.arange(4)[None])
    assert facade.compiled_entry_count == 0
    with pytest.raises(ValueError, match="backend"):
        g.compile_gemma4_mi355x_layer(glob, backend="nonsense")


def _cache(cfg, max_len):
    cache = cu.StaticCache(config=cfg, max_cache_len=max_len)
    cache.early_initialization(1, [16 if t == "sliding_attention" else 4 for t in cfg.layer_types],
                               [256 if t == "sliding_attention" else 512 for t in cfg.layer_types],
                               torch.bfloat16, torch.device("cpu"))
    return cache


def test_static_cache_binding_checks_layer_classes_and_capacity(modules):
    cfg, local, glob = modules
    cache = _cache(cfg, 1100)
    f = g.compile_gemma4_mi355x_static_cache_decode(glob, cache)
    assert isinstance(f, g.Gemma4MI355XCompiledStaticCacheDecodeFacade)
    f2 = g.compile_gemma4_mi355x_static_cache_decode(local, cache)
    assert isinstance(f2, g.Gemma4MI355XCompiledLocalStaticCacheDecodeFacade)
    h = torch.zeros(1, 1, 5376, dtype=torch.bfloat16)
    rope = (torch.ones(1, 1, 512, dtype=torch.bfloat16), torch.zeros(1, 1, 512, dtype=torch.bfloat16))
    with torch.no_grad(), pytest.raises(UnsupportedMI355XPath, match="CUDA"):
        f(h, rope, position_ids=torch.zeros(1, 1, dtype=torch.int64))
    # a sliding layer shorter than the 1024-token window is not the locked cache
    with pytest.raises(UnsupportedMI355XPath, match="1024-slot"):
        g.compile_gemma4_mi355x_static_cache_decode(local, _cache(cfg, 96))
    with pytest.raises(UnsupportedMI355XPath, match="StaticCache"):
        g.compile_gemma4_mi355x_static_cache_decode(glob, object())
    # rebinding the layer's storage is detected before a call
    cache.layers[5].keys = cache.layers[5].keys.clone()
    with torch.no_grad(), pytest.raises(UnsupportedMI355XPath, match="replaced|CUDA"):
        f(h, rope, position_ids=torch.zeros(1, 1, dtype=torch.int64))
