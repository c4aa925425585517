"""The torch custom-op layer on the CPU (no kernel runs): every op registers
under torch.ops.pe with the schema the boundary needs (mutated caches, scratch
and status declared), and its fake implementation gives the output shapes and
dtypes a trace sees."""

from types import SimpleNamespace

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from parallel_eagle_amd import ops


@pytest.fixture(scope="module")
def pe_ops():
    ops.register_torch_ops()
    ops.register_torch_ops()  # idempotent
    return torch.ops.pe


def _schema(op) -> str:
    return str(op.default._schema)


def test_schemas_declare_every_mutation(pe_ops):
    s = _schema(pe_ops.verify_pass)
    for name in ("k_cache", "v_cache", "workspace", "status"):
        assert f"!) {name}" in s, (name, s)
    assert "!) tree_bits" not in s and "!) input_ids" not in s
    assert "Tensor(a!) status" in _schema(pe_ops.tree_masks)
    assert "Tensor(a!) scratch" in _schema(pe_ops.accept_tree)
    assert "!) k_cache" in _schema(pe_ops.kv_compact) and "!) v_cache" in _schema(pe_ops.kv_compact)
    assert "!) accept_out" not in _schema(pe_ops.kv_compact)
    assert "!) status" in _schema(pe_ops.kv_gather)


def test_fake_implementations_give_output_shapes(pe_ops):
    stub = SimpleNamespace(shape=SimpleNamespace(vocab=32000), dtype=torch.bfloat16, feature_dim=3 * 4096)
    h = ops.register_model(stub)
    assert ops.register_model(stub) == h
    with FakeTensorMode():
        dev = "cuda"
        par = torch.empty(26, dtype=torch.int32, device=dev)
        st = torch.empty(4, dtype=torch.int32, device=dev)
        bits, pos, dep = pe_ops.tree_masks(par, 2048, 1, st)
        assert (bits.shape, bits.dtype, pos.shape, pos.dtype, dep.dtype) == (
            (26, 1), torch.int64, (26,), torch.int64, torch.int32)
        ids = torch.empty(26, dtype=torch.int64, device=dev)
        k = torch.empty((32, 32, 2112, 128), dtype=torch.bfloat16, device=dev)
        ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)
        lg, fu = pe_ops.verify_pass(h, ids, pos, bits, k, torch.empty_like(k), 2048, ws, st)
        assert (lg.shape, lg.dtype, fu.shape) == ((26, 32000), torch.bfloat16, (26, 12288))
        root = torch.empty(32000, dtype=torch.bfloat16, device=dev)
        out = pe_ops.accept_tree(root, lg, ids, par, torch.empty(28, dtype=torch.int32, device=dev))
        assert (out.shape, out.dtype) == ((28,), torch.int32)
        assert pe_ops.kv_compact(k, torch.empty_like(k), 2048, out) is None
        assert pe_ops.argmax_rows(lg).shape == (26,)
        x = torch.empty((26, 4096), dtype=torch.bfloat16, device=dev)
        assert pe_ops.rmsnorm(x, torch.empty(4096, dtype=torch.bfloat16, device=dev), 1e-5).shape == (26, 4096)
        assert pe_ops.dense_linear(x, torch.empty(4096 * 512, dtype=torch.bfloat16, device=dev), 512).shape == (26, 512)


def test_unknown_model_handle_is_refused(pe_ops):
    with FakeTensorMode(), pytest.raises(ValueError, match="no target registered"):
        ids = torch.empty(3, dtype=torch.int64, device="cuda")
        k = torch.empty((1, 1, 8, 64), device="cuda")
        pe_ops.verify_pass(10 ** 6, ids, ids, torch.empty((3, 1), dtype=torch.int64, device="cuda"), k, k, 0,
                           torch.empty(8, dtype=torch.uint8, device="cuda"), torch.empty(4, dtype=torch.int32,
                                                                                           device="cuda"))
