"""The vLLM patches ``register_backend`` installs (reference
``vllm_plugin/plugin.py:32-61``, ``:125-491``), exercised against stand-in
vLLM modules on the CPU: vLLM is not installed here, so each test builds the
few classes and functions a patch touches, with vLLM's names and call
signatures, in ``sys.modules`` for the duration of the test.
"""
import dataclasses
import os
import sys
import types

import pytest
import torch


def _mod(name, **attrs):
    m = types.ModuleType(name)
    for k, v in attrs.items():
        setattr(m, k, v)
    return m


@dataclasses.dataclass(frozen=True)
class FullAttentionSpec:
    block_size: int
    num_kv_heads: int
    head_size: int
    dtype: torch.dtype = torch.bfloat16

    @property
    def page_size_bytes(self) -> int:
        return 2 * self.block_size * self.num_kv_heads * self.head_size * torch.finfo(self.dtype).bits // 8


@dataclasses.dataclass(frozen=True)
class SlidingWindowSpec(FullAttentionSpec):
    sliding_window: int = 1024


@dataclasses.dataclass(frozen=True)
class TQFullAttentionSpec(FullAttentionSpec):
    head_size_v: int = 0
    tq_slot_size: int = 0

    @property
    def page_size_bytes(self) -> int:
        return self.block_size * self.num_kv_heads * self.tq_slot_size


class Attention:
    def __init__(self, head_size, kv_cache_dtype, spec):
        self.head_size = head_size
        self.kv_cache_dtype = kv_cache_dtype
        self._spec = spec

    def get_kv_cache_spec(self, vllm_config=None):
        return self._spec


def _stock_unify(kv_cache_spec):
    if len({s.page_size_bytes for s in kv_cache_spec.values()}) > 1:
        raise NotImplementedError("stock vLLM: page sizes differ")
    return kv_cache_spec


class TurboQuantConfig:
    @staticmethod
    def get_boundary_skip_layers(num_layers, n=2):
        return list(range(n)) + list(range(num_layers - n, num_layers))


@dataclasses.dataclass
class EngineArgs:
    model: str = "m"
    kv_cache_dtype: str = "auto"
    additional_config: dict = dataclasses.field(default_factory=dict)
    seen_dtype: str = ""

    def __post_init__(self):
        # vLLM validates the cache dtype against its Literal of stock presets here
        if self.kv_cache_dtype not in ("auto", "turboquant_3bit_nc", "turboquant_k3v4_nc", "turboquant_4bit_nc"):
            raise ValueError(f"invalid cache dtype {self.kv_cache_dtype}")
        self.seen_dtype = self.kv_cache_dtype


class _Enum:
    TURBOQUANT = "TURBOQUANT"


@pytest.fixture
def fake_vllm(monkeypatch):
    """Stand-in vLLM modules, fresh per test (patched attributes die with them)."""
    registered = {}
    attn_cls = type("Attention", (Attention,), {})
    tqc = type("TurboQuantConfig", (TurboQuantConfig,), {})
    ea = dataclasses.dataclass(type("EngineArgs", (EngineArgs,), {}))
    mods = {
        "vllm": _mod("vllm"),
        "vllm.v1": _mod("vllm.v1"),
        "vllm.v1.attention": _mod("vllm.v1.attention"),
        "vllm.v1.attention.backends": _mod("vllm.v1.attention.backends"),
        "vllm.v1.attention.backends.registry": _mod(
            "vllm.v1.attention.backends.registry", AttentionBackendEnum=_Enum,
            register_backend=lambda enum, path: registered.__setitem__(enum, path)),
        "vllm.v1.kv_cache_interface": _mod("vllm.v1.kv_cache_interface", FullAttentionSpec=FullAttentionSpec,
                                           SlidingWindowSpec=SlidingWindowSpec,
                                           TQFullAttentionSpec=TQFullAttentionSpec),
        "vllm.v1.core": _mod("vllm.v1.core"),
        "vllm.v1.core.kv_cache_utils": _mod("vllm.v1.core.kv_cache_utils",
                                            unify_kv_cache_spec_page_size=_stock_unify),
        "vllm.model_executor": _mod("vllm.model_executor"),
        "vllm.model_executor.layers": _mod("vllm.model_executor.layers"),
        "vllm.model_executor.layers.attention": _mod("vllm.model_executor.layers.attention"),
        "vllm.model_executor.layers.attention.attention": _mod(
            "vllm.model_executor.layers.attention.attention", Attention=attn_cls),
        "vllm.model_executor.layers.quantization": _mod("vllm.model_executor.layers.quantization"),
        "vllm.model_executor.layers.quantization.turboquant": _mod(
            "vllm.model_executor.layers.quantization.turboquant"),
        "vllm.model_executor.layers.quantization.turboquant.config": _mod(
            "vllm.model_executor.layers.quantization.turboquant.config", TurboQuantConfig=tqc),
        "vllm.engine": _mod("vllm.engine"),
        "vllm.engine.arg_utils": _mod("vllm.engine.arg_utils", EngineArgs=ea),
    }
    parent_links = {
        "vllm.model_executor.layers.attention": ("attention", "vllm.model_executor.layers.attention.attention"),
        "vllm.v1.core": ("kv_cache_utils", "vllm.v1.core.kv_cache_utils"),
    }
    for name, mod in mods.items():
        monkeypatch.setitem(sys.modules, name, mod)
    for parent, (attr, child) in parent_links.items():
        setattr(mods[parent], attr, mods[child])
    for k in ("TURBOQUANT_KEY_BITS", "TURBOQUANT_VALUE_BITS", "TURBOQUANT_BOUNDARY_PROTECT",
              "TURBOQUANT_V_ROTATE", "TURBOQUANT_KIND"):
        monkeypatch.setenv(k, "")  # records the original value (set or not), restored at teardown
        monkeypatch.delenv(k)
    return types.SimpleNamespace(mods=mods, registered=registered, Attention=attn_cls, TQC=tqc, EA=ea)


def test_register_backend_installs_every_patch(fake_vllm):
    from fused_turboquant.vllm_plugin import plugin
    assert plugin.register_backend() is True
    assert fake_vllm.registered["TURBOQUANT"].endswith("v1_backend.FusedTurboQuantV1Backend")
    assert plugin._patched(fake_vllm.Attention.get_kv_cache_spec)
    assert plugin._patched(fake_vllm.mods["vllm.v1.core.kv_cache_utils"].unify_kv_cache_spec_page_size)
    assert plugin._patched(fake_vllm.EA.__post_init__)
    # boundary protection is on by default: vLLM's skip list stays
    assert fake_vllm.TQC.get_boundary_skip_layers(10) == [0, 1, 8, 9]
    # idempotent: a second registration wraps nothing twice
    spec_fn = fake_vllm.Attention.get_kv_cache_spec
    post = fake_vllm.EA.__post_init__
    assert plugin.register_backend() is True
    assert fake_vllm.Attention.get_kv_cache_spec is spec_fn and fake_vllm.EA.__post_init__ is post


def test_kv_cache_spec_uses_the_backends_slot_size(fake_vllm, monkeypatch):
    from fused_turboquant.vllm_plugin import plugin
    from fused_turboquant.vllm_plugin.v1_backend import FusedTurboQuantV1Backend as B
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "0")
    assert plugin.patch_kv_cache_spec()
    A = fake_vllm.Attention
    for spec in (FullAttentionSpec(16, 8, 128), SlidingWindowSpec(16, 8, 128),
                 TQFullAttentionSpec(16, 8, 128, head_size_v=128, tq_slot_size=104)):
        out = A(128, "turboquant_k4v2_nc", spec).get_kv_cache_spec()
        assert isinstance(out, TQFullAttentionSpec) and out.dtype == torch.uint8
        assert out.tq_slot_size == B._slot_size_for(128, "turboquant_k4v2_nc") == 256
        # vLLM's page bytes == the bytes of the backend's cache shape for one block
        shape = B.get_kv_cache_shape(1, 16, 8, 128, "turboquant_k4v2_nc")
        assert out.page_size_bytes == shape[1] * shape[2] * shape[3]
    raw = FullAttentionSpec(16, 8, 128)
    assert A(128, "auto", raw).get_kv_cache_spec() is raw  # other backends' layers untouched


def test_unify_page_sizes_widens_by_integer_ratio(fake_vllm):
    from fused_turboquant.vllm_plugin import plugin
    assert plugin.patch_unify_page_size()
    unify = fake_vllm.mods["vllm.v1.core.kv_cache_utils"].unify_kv_cache_spec_page_size
    spec = {"full": TQFullAttentionSpec(16, 8, 512, tq_slot_size=1024),
            "slide": TQFullAttentionSpec(16, 8, 256, tq_slot_size=256)}
    out = unify(spec)
    assert out["full"] is spec["full"]
    assert out["slide"].block_size == 64 and out["slide"].page_size_bytes == spec["full"].page_size_bytes
    same = {"a": spec["full"]}
    assert unify(same) is same
    with pytest.raises(NotImplementedError):
        unify({"a": TQFullAttentionSpec(16, 8, 128, tq_slot_size=256),
               "b": TQFullAttentionSpec(16, 8, 128, tq_slot_size=96)})


def test_boundary_skip_layers_off(fake_vllm, monkeypatch):
    from fused_turboquant.vllm_plugin import plugin
    assert plugin.patch_boundary_skip_layers() is False  # protection on: vLLM's default stays
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "0")
    assert plugin.patch_boundary_skip_layers() is True
    assert fake_vllm.TQC.get_boundary_skip_layers(32) == []
    assert plugin.patch_boundary_skip_layers() is True  # idempotent


def test_engine_args_alias_rewritten_before_validation(fake_vllm, monkeypatch):
    from fused_turboquant.vllm_plugin import plugin
    with pytest.raises(ValueError):  # without the patch vLLM rejects the alias
        fake_vllm.EA(kv_cache_dtype="turboquant_k3v2_nc")
    assert plugin.patch_engine_args()
    ea = fake_vllm.EA(kv_cache_dtype="turboquant_k3v2_nc",
                      additional_config={"turboquant": {"v_rotate": True, "kind": "planar"}})
    assert ea.seen_dtype == "turboquant_3bit_nc" == ea.kv_cache_dtype
    assert os.environ["TURBOQUANT_KEY_BITS"] == "3" and os.environ["TURBOQUANT_VALUE_BITS"] == "2"
    assert os.environ["TURBOQUANT_V_ROTATE"] == "1" and os.environ["TURBOQUANT_KIND"] == "planar"
    # the effective widths reach the backend through host_preset
    assert plugin.host_preset(ea.kv_cache_dtype) == ("turboquant_3bit_nc", 3, 2)
    # 1-bit aliases map the same way; explicit environment values win
    monkeypatch.setenv("TURBOQUANT_VALUE_BITS", "4")
    monkeypatch.setenv("TURBOQUANT_KEY_BITS", "1")
    ea = fake_vllm.EA(kv_cache_dtype="turboquant_k1v4_nc")
    assert ea.kv_cache_dtype == "turboquant_k3v4_nc"
    assert plugin.host_preset(ea.kv_cache_dtype) == ("turboquant_k3v4_nc", 1, 4)
    # stock presets and non-TurboQuant dtypes pass through
    assert fake_vllm.EA(kv_cache_dtype="auto").seen_dtype == "auto"


def test_patches_are_no_ops_without_vllm():
    from fused_turboquant.vllm_plugin import plugin
    try:
        import vllm  # noqa: F401
        pytest.skip("vLLM is installed")
    except ImportError:
        pass
    assert plugin.patch_kv_cache_spec() is False
    assert plugin.patch_unify_page_size() is False
    assert plugin.patch_engine_args() is False
    assert plugin.patch_cache_dtype_validation() is False
