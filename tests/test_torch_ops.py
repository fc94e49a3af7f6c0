"""torch.ops.fused_tq: the operator library loads without a GPU, every
operator has the schema the package calls it with, and the shape-only (fake)
implementations give the shapes and dtypes of the real ones, so torch.compile
and other tracers see through the calls."""
import pytest
import torch

from conftest import ROOT  # noqa: F401  (puts the package on sys.path)


def _ops():
    from fused_turboquant import _lib, _ops
    import os
    if not (os.path.exists(_lib.LIB_PATH) and os.path.exists(_ops.OPS_PATH)):
        import __graft_entry__
        __graft_entry__.build()
    return _ops.ops()


def test_operator_schemas():
    ops = _ops()
    want = {
        "encode": "encode(Tensor x, Tensor signs, Tensor boundaries, int bits, int codebook_class) -> (Tensor, Tensor)",
        "decode": "decode(Tensor packed, Tensor norms, Tensor levels, Tensor signs, int bits, int d, "
                  "ScalarType out_dtype) -> Tensor",
        "rht": "rht(Tensor x, Tensor signs, bool inverse, ScalarType out_dtype) -> Tensor",
    }
    for name, schema in want.items():
        assert str(getattr(ops, name).default._schema) == "fused_tq::" + schema
    # in-place operators name the tensors they write
    assert "Tensor(a!) kv_cache" in str(ops.v1_store.default._schema)
    assert "Tensor(b!) out" in str(ops.v1_decode_attention.default._schema)
    assert "Tensor(c!)? lse" in str(ops.raw_decode_attention.default._schema)
    assert "bool fp32_operands" in str(ops.paged_decode_attention.default._schema)


def test_fake_implementations_give_shapes():
    from torch._subclasses.fake_tensor import FakeTensorMode
    ops = _ops()
    with FakeTensorMode():
        x = torch.empty(5, 7, 128, dtype=torch.bfloat16, device="cuda")
        s = torch.empty(128, device="cuda")
        b = torch.empty(9, device="cuda")
        packed, norms = ops.encode(x, s, b, 3, 0)
        assert packed.shape == (5, 7, 48) and packed.dtype == torch.uint8
        assert norms.shape == (5, 7) and norms.dtype == torch.float16
        dec = ops.decode(packed, norms, torch.empty(8, device="cuda"), s, 3, 128, torch.bfloat16)
        assert dec.shape == (5, 7, 128) and dec.dtype == torch.bfloat16
        r = ops.rht(x, s, True, torch.float32)
        assert r.shape == x.shape and r.dtype == torch.float32
        kp, kn, vp, vn = ops.encode_kv(x, x, s, b, 3, 0)
        for p, n in ((kp, kn), (vp, vn)):
            assert p.shape == (5, 7, 48) and p.dtype == torch.uint8
            assert n.shape == (5, 7) and n.dtype == torch.float16


def test_cpu_tensors_rejected_by_the_package():
    from fused_turboquant import TurboQuantMSE
    from fused_turboquant._lib import FusedTQError
    tq = TurboQuantMSE(128, bits=3)
    with pytest.raises(FusedTQError):
        tq.encode(torch.zeros(4, 128))
