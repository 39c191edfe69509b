"""Host logic of the drop-in router (CPU): without a controller router_attention is exactly SDPA
(STRATA_KV.py:499-504); with one it forwards to controller.attend and refuses sliding-window and
soft-capped attention (508-509); routed() restores the previous controller (517-523)."""
from types import SimpleNamespace

import pytest
import torch


def test_router_without_controller_is_sdpa():
    import kvq
    g = torch.Generator().manual_seed(0)
    B, Hq, Hkv, T, d = 1, 8, 2, 12, 16
    q = torch.randn(B, Hq, T, d, generator=g)
    k = torch.randn(B, Hkv, T, d, generator=g)
    v = torch.randn(B, Hkv, T, d, generator=g)
    module = SimpleNamespace(layer_idx=0, scaling=d ** -0.5, num_key_value_groups=Hq // Hkv, is_causal=True,
                             training=False)
    out, _ = kvq.router_attention(module, q, k, v, None, scaling=d ** -0.5)
    ref = torch.nn.functional.scaled_dot_product_attention(
        q, k.repeat_interleave(Hq // Hkv, 1), v.repeat_interleave(Hq // Hkv, 1), is_causal=True,
        scale=d ** -0.5).transpose(1, 2)
    assert torch.allclose(out, ref, atol=1e-6)


def test_router_forwards_and_refuses_sliding_window():
    import kvq

    class Ctl:
        def attend(self, module, q, k, v, mask, kwargs):
            return ("called", kwargs.get("scaling")), None

    module = SimpleNamespace(layer_idx=3, scaling=0.5)
    ctl = Ctl()
    assert kvq.Router.active is None
    with kvq.routed(ctl):
        out, _ = kvq.router_attention(module, None, None, None, None, scaling=0.25)
        assert out == ("called", 0.25)
        with pytest.raises(RuntimeError, match="sliding-window"):
            kvq.router_attention(module, None, None, None, None, sliding_window=4096)
        with pytest.raises(RuntimeError, match="soft-capped"):
            kvq.router_attention(module, None, None, None, None, softcap=30.0)
        with pytest.raises(RuntimeError):
            kvq.router_attention(SimpleNamespace(layer_idx=1, sliding_window=512), None, None, None, None)
    assert kvq.Router.active is None


def test_register_with_transformers():
    import kvq
    from transformers import AttentionInterface
    name = kvq.register()
    assert AttentionInterface._global_mapping[name] is kvq.router_attention
