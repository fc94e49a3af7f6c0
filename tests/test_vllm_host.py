"""Host logic of the vLLM TURBOQUANT backend surface (no GPU): cache-dtype
presets and per-K/V overrides (reference ``vllm_plugin/plugin.py:380-412``),
the cache shape vLLM allocates (``v1_backend.py:171-220``), dtype support and
the Impl's refusal of features this build does not carry."""
import pytest

from fused_turboquant import vllm_plugin as vp

B = vp.FusedTurboQuantV1Backend


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    for k in ("TURBOQUANT_KEY_BITS", "TURBOQUANT_VALUE_BITS", "TURBOQUANT_V_ROTATE",
              "TURBOQUANT_V_LLOYD_MAX", "TURBOQUANT_BOUNDARY_PROTECT", "TURBOQUANT_KIND"):
        monkeypatch.setenv(k, "")  # records the original value, restored at teardown
        monkeypatch.delenv(k)


@pytest.mark.parametrize("dt,want", [
    ("turboquant_3bit_nc", ("turboquant_3bit_nc", 3, 3)),
    ("turboquant_k3v4_nc", ("turboquant_k3v4_nc", 3, 4)),
    ("turboquant_4bit_nc", ("turboquant_4bit_nc", 4, 4)),
    ("turboquant_k4v2_nc", ("turboquant_4bit_nc", 4, 2)),
    ("turboquant_k2v4_nc", ("turboquant_k3v4_nc", 2, 4)),
    ("turboquant_k2v2_nc", ("turboquant_3bit_nc", 2, 2)),
    ("turboquant_k3v3_nc", ("turboquant_3bit_nc", 3, 3)),
    ("turboquant_k1v2_nc", ("turboquant_3bit_nc", 1, 2)),
    ("turboquant_k1v4_nc", ("turboquant_k3v4_nc", 1, 4)),
    ("turboquant_k4v1_nc", ("turboquant_4bit_nc", 4, 1)),
    ("turboquant_k1v1_nc", ("turboquant_3bit_nc", 1, 1)),
])
def test_host_preset(dt, want):
    assert vp.host_preset(dt) == want


def test_host_preset_env_override(monkeypatch):
    monkeypatch.setenv("TURBOQUANT_KEY_BITS", "2")
    monkeypatch.setenv("TURBOQUANT_VALUE_BITS", "3")
    assert vp.host_preset("turboquant_4bit_nc") == ("turboquant_4bit_nc", 2, 3)
    monkeypatch.setenv("TURBOQUANT_KEY_BITS", "4")
    with pytest.raises(ValueError, match="exceeds the slot"):
        vp.host_preset("turboquant_3bit_nc")


@pytest.mark.parametrize("dt", ["fp8", "turboquant_5bit_nc", "turboquant_k5v2_nc", "turboquant_k0v2_nc", "auto"])
def test_host_preset_rejects(dt):
    with pytest.raises(ValueError):
        vp.host_preset(dt)


@pytest.mark.parametrize("dt,protect,slot", [
    # K3V3 d128: 48 + 2 + 48 + 4 = 102 bytes -> 128; K3V4: 118 -> 128; K4V4: 134 -> 256
    ("turboquant_3bit_nc", "0", 128), ("turboquant_k3v4_nc", "0", 128), ("turboquant_4bit_nc", "0", 256),
    ("turboquant_k4v2_nc", "0", 256), ("turboquant_k2v3_nc", "0", 128),
    # boundary layers share the allocation: at least 2 * head_size
    ("turboquant_3bit_nc", "1", 256), ("turboquant_4bit_nc", "1", 256),
])
def test_kv_cache_shape(monkeypatch, dt, protect, slot):
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", protect)
    assert B.get_kv_cache_shape(100, 16, 8, 128, dt) == (100, 16, 8, slot)


def test_kv_cache_shape_d64_d256(monkeypatch):
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "0")
    # d64 K3V3: 24 + 2 + 24 + 4 = 54 -> 64; d256 K4V4: 128 + 2 + 128 + 4 = 262 -> 512
    assert B.get_kv_cache_shape(4, 16, 2, 64, "turboquant_3bit_nc")[-1] == 64
    assert B.get_kv_cache_shape(4, 16, 2, 256, "turboquant_4bit_nc")[-1] == 512


def test_backend_surface():
    assert B.get_name() == "TURBOQUANT"
    assert B.get_impl_cls() is vp.FusedTurboQuantV1Impl
    assert B.accept_output_buffer and not B.forward_includes_kv_cache_update
    assert 16 in B.get_supported_kernel_block_sizes()
    assert B.supports_kv_cache_dtype("turboquant_k4v2_nc")
    assert B.supports_kv_cache_dtype("turboquant_3bit_nc")
    assert not B.supports_kv_cache_dtype("fp8_e4m3")
    assert B.supports_head_size(128) and B.supports_head_size(64) and B.supports_head_size(256)
    assert not B.supports_head_size(96)


def test_impl_init_and_refusals(monkeypatch):
    monkeypatch.setenv("TURBOQUANT_V_ROTATE", "1")
    im = vp.FusedTurboQuantV1Impl(32, 128, 128 ** -0.5, 8, kv_cache_dtype="turboquant_k4v2_nc")
    assert (im.key_bits, im.value_bits, im.v_rotate, im.num_kv_groups) == (4, 2, True, 4)
    mk = lambda **kw: vp.FusedTurboQuantV1Impl(**{**dict(num_heads=8, head_size=128, scale=0.1,
                                                         num_kv_heads=2, kv_cache_dtype="turboquant_3bit_nc"), **kw})
    with pytest.raises(NotImplementedError):
        mk(alibi_slopes=[1.0] * 8)
    with pytest.raises(NotImplementedError):
        mk(kv_sharing_target_layer_name="layers.0")
    # sliding windows are applied (a Gemma-style layer: head 256, window 512); soft-capping is refused
    gem = mk(head_size=256, num_heads=8, num_kv_heads=4, sliding_window=512, kv_cache_dtype="turboquant_k3v4_nc")
    assert gem.sliding_window == 512 and gem.head_size == 256
    assert mk(sliding_window=None).sliding_window is None
    with pytest.raises(ValueError):
        mk(sliding_window=0)
    with pytest.raises(NotImplementedError):
        mk(logits_soft_cap=30.0)
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL", "1")
    with pytest.raises(NotImplementedError):
        mk(sliding_window=128)
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL", "0")
    with pytest.raises(NotImplementedError):
        mk(head_size=96)
    assert mk(head_size=64).head_size == 64 and mk(head_size=256).head_size == 256
    with pytest.raises(ValueError):
        mk(num_heads=8, num_kv_heads=3)
    with pytest.raises(ValueError):
        mk(num_heads=64, num_kv_heads=2)


def test_apply_additional_config(monkeypatch):
    class EA:
        additional_config = {"turboquant": {"v_rotate": True, "key_bits": 2, "boundary_protect": False}}
    monkeypatch.setenv("TURBOQUANT_KEY_BITS", "3")  # explicit environment wins
    vp.apply_additional_config(EA())
    import os
    assert os.environ["TURBOQUANT_V_ROTATE"] == "1"
    assert os.environ["TURBOQUANT_KEY_BITS"] == "3"
    assert os.environ["TURBOQUANT_BOUNDARY_PROTECT"] == "0"
    assert not vp.boundary_protect_enabled()


def test_register_without_vllm():
    try:
        import vllm  # noqa: F401
        pytest.skip("vLLM is installed")
    except ImportError:
        pass
    assert vp.register_backend() is False


@pytest.mark.parametrize("raw,want", [("0", "off"), ("off", "off"), ("1", "fp16"), ("bf16", "fp16"),
                                      ("FP16", "fp16"), ("fp8", "fp8"), ("2", 2), ("3", 3), ("4", 4), ("8", 8)])
def test_boundary_protect_mode(monkeypatch, raw, want):
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", raw)
    assert vp.boundary_protect_mode() == want
    assert vp.boundary_protect_enabled() == (want != "off")


@pytest.mark.parametrize("raw", ["5", "yes please", "16"])
def test_boundary_protect_mode_rejects(monkeypatch, raw):
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", raw)
    with pytest.raises(ValueError):
        vp.boundary_protect_mode()


def test_boundary_layer_impl_modes(monkeypatch):
    mk = lambda: vp.FusedTurboQuantV1Impl(32, 128, 0.1, 8, kv_cache_dtype="auto")
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "1")   # default: raw fp16 slots
    im = mk()
    assert im._is_raw and im.preset == "raw_fp16" and not im.v_rotate
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "3")   # TurboQuant codes at 3 bits in the fp16 slot
    im = mk()
    assert not im._is_raw and (im.key_bits, im.value_bits) == (3, 3)
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "8")   # 8-bit Lloyd-Max K, 8-bit V
    im = mk()
    assert (im.key_bits, im.value_bits, im.key_fp8, im.preset) == (8, 8, False, "boundary_8bit")
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "fp8")  # fp8 keys, 8-bit V
    im = mk()
    assert (im.key_bits, im.value_bits, im.key_fp8, im.preset) == (8, 8, True, "boundary_fp8")
    # both fit the fp16-sized slot vLLM gives boundary layers (reference README: 262 bytes at d=128)
    from fused_turboquant import v1
    assert v1.slot_bytes(128, 8, 8) == 262 and v1.slot_bytes(128, 8, 8, key_fp8=True) == 260 <= 4 * 128
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "0")
    with pytest.raises(NotImplementedError):
        mk()
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "fp16")
    with pytest.raises(ValueError):  # raw decode kernel: GQA group <= 8
        vp.FusedTurboQuantV1Impl(32, 128, 0.1, 2, kv_cache_dtype="bfloat16")
    # the boundary layer's slot (bf16 elements) holds K|V in fp16: 4 * head_size bytes
    assert B.get_kv_cache_shape(10, 16, 8, 128, "auto")[-1] * 2 == 4 * 128


def test_defer_prefill_flag_and_capacity(monkeypatch):
    from fused_turboquant import vllm_plugin as vp
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "0")
    monkeypatch.delenv("TURBOQUANT_DEFER_PREFILL", raising=False)
    impl = vp.FusedTurboQuantV1Impl(32, 128, 0.088, 8, kv_cache_dtype="turboquant_3bit_nc")
    assert not impl.defer_prefill
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL", "1")
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL_CAPACITY", "4096")
    impl = vp.FusedTurboQuantV1Impl(32, 128, 0.088, 8, kv_cache_dtype="turboquant_3bit_nc")
    assert impl.defer_prefill and impl._prefix_capacity == 4096
    # raw fp16 boundary layers never defer (reference: _store_raw_kv returns first)
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "fp16")
    raw = vp.FusedTurboQuantV1Impl(32, 128, 0.088, 8, kv_cache_dtype="auto")
    assert not raw.defer_prefill
    monkeypatch.setenv("TURBOQUANT_BOUNDARY_PROTECT", "0")
    monkeypatch.setenv("TURBOQUANT_DEFER_PREFILL_CAPACITY", "1")
    with pytest.raises(ValueError):
        vp.FusedTurboQuantV1Impl(32, 128, 0.088, 8, kv_cache_dtype="turboquant_3bit_nc")


def test_additional_config_maps_defer_and_lloyd_keys():
    from fused_turboquant.vllm_plugin import plugin
    assert plugin.TQ_CONFIG_ENV_MAP["defer_prefill"] == "TURBOQUANT_DEFER_PREFILL"
    assert plugin.TQ_CONFIG_ENV_MAP["v_lloyd_max"] == "TURBOQUANT_V_LLOYD_MAX"


def test_kind_env_registered_and_unknown(monkeypatch):
    """TURBOQUANT_KIND: every name the reference registers builds (rht,
    planar, rotor, iso_fast, iso_full); others raise ValueError as the
    reference's registry lookup does (v1_backend.py:516-523), matched as given
    (no case folding)."""
    from fused_turboquant import vllm_plugin as vp
    for k in ("planar", "rotor", "iso_fast", "iso_full", "rht"):
        monkeypatch.setenv("TURBOQUANT_KIND", k)
        assert vp.FusedTurboQuantV1Impl(32, 128, 128 ** -0.5, 8, kv_cache_dtype="turboquant_k4v2_nc").kind == k
    for k in ("iso", "bogus", "Planar", "RHT"):
        monkeypatch.setenv("TURBOQUANT_KIND", k)
        with pytest.raises(ValueError, match="not registered"):
            vp.FusedTurboQuantV1Impl(32, 128, 128 ** -0.5, 8, kv_cache_dtype="turboquant_k4v2_nc")
