"""Host-side argument checks of tops.ops.simple_gla (no kernel launch; CPU)."""
import pytest
import torch


def _t(*shape):
    return torch.zeros(*shape)


def test_chunk_mode_rejects_per_token_gate_like_the_reference():
    """tops/ops/simple_gla/__init__.py:92-102: mode='chunk' raises on g, reverse, cu_seqlens."""
    from tops.ops.simple_gla import simple_gla
    q = _t(1, 8, 2, 16)
    v = _t(1, 8, 2, 16)
    gg = _t(2)
    with pytest.raises(ValueError):
        simple_gla(q, q, v, g=_t(1, 8, 2), g_gamma=gg, mode="chunk")
    with pytest.raises(ValueError):
        simple_gla(q, q, v, g_gamma=gg, reverse=True, mode="chunk")
    with pytest.raises(ValueError):
        simple_gla(q, q, v, g_gamma=gg, cu_seqlens_cpu=[0, 8], mode="fused_chunk")
    with pytest.raises(ValueError):
        simple_gla(q, q, v, g_gamma=gg, mode="bogus")


def test_both_gates_rejected():
    from tops.ops.simple_gla import chunk_simple_gla
    q = _t(1, 8, 2, 16)
    with pytest.raises(ValueError):
        chunk_simple_gla(q, q, q, _t(2), g=_t(1, 8, 2))


def test_cpu_tensors_fail_loudly():
    """No CPU fallback: the HIP library is the only compute path."""
    from tops.ops.simple_gla import chunk_simple_gla
    from tops._native import TopsError
    q = _t(1, 8, 2, 16)
    with pytest.raises(TopsError):
        chunk_simple_gla(q, q, q, _t(2))


def test_inference_inputs_detach_only_without_grad_mode():
    """Under no_grad an autograd Function still sees needs_input_grad = True for inputs that
    require grad; the ops detach their inputs there so that no backward state is kept."""
    import torch
    from tops.utils import inference_inputs
    x = torch.ones(3, requires_grad=True)
    a, b = inference_inputs(x, None)
    assert a is x and b is None
    with torch.no_grad():
        a, b, c = inference_inputs(x, None, 2.0)
    assert not a.requires_grad and a.data_ptr() == x.data_ptr() and b is None and c == 2.0
