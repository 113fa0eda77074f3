"""Kernel selection and registration against a stand-in vLLM module tree (vLLM is not installed).

The stand-in holds only what the plugin binds to: the MxFp4LinearKernel ABC and its layer config
(vllm.model_executor.kernels.linear.mxfp4.base), the priority registry _POSSIBLE_MXFP4_KERNELS of
vllm.model_executor.kernels.linear that init_mxfp4_linear_kernel reads, current_platform._enum,
the kMxfp4Dynamic activation key and AITER's asm-fp4 switch. The checks follow the reference's
selection contract: sly/patch_quark_mxfp4.py:76-103 puts the plugin at index 0 of the platform's
list, is_supported declines unless the switch is set, the library loads and the GPU is the one the
kernels are built for (sly/mxfp4/radiance_mxfp4.py:1019-1025), and can_implement declines any
other activation key and AITER's asm layout (:1027-1037). No GPU call is made."""
import sys
import types

import pytest

from vllm_sly_radiance_amd import _native
from vllm_sly_radiance_amd import radiance_mxfp4 as R


class _Key:
    def __init__(self, name):
        self.name = name

    def __repr__(self):
        return self.name


K_MXFP4_DYNAMIC = _Key("kMxfp4Dynamic")
K_OTHER = _Key("kFp8StaticTensorSym")
ROCM = "PlatformEnum.ROCM"


class _OtherKernel:
    """A kernel vLLM already lists for the platform (stands in for AITER's / Triton's)."""


@pytest.fixture
def fake_vllm(monkeypatch):
    """Install the stand-in tree in sys.modules and rebuild the plugin class on it."""
    mods = {}

    def mod(name, **attrs):
        m = types.ModuleType(name)
        m.__dict__.update(attrs)
        mods[name] = m
        return m

    class MxFp4LinearLayerConfig:
        def __init__(self, activation_quant_key):
            self.activation_quant_key = activation_quant_key

    class MxFp4LinearKernel:
        def __init__(self, c):
            self.config = c

    asm = types.SimpleNamespace(enabled=False)

    class _AiterOps:
        @staticmethod
        def is_asm_fp4_gemm_dynamic_quant_enabled():
            return asm.enabled

    mod("vllm")
    mod("vllm.platforms", current_platform=types.SimpleNamespace(_enum=ROCM))
    mod("vllm._aiter_ops", rocm_aiter_ops=_AiterOps)
    mod("vllm.model_executor")
    mod("vllm.model_executor.kernels")
    registry = mod("vllm.model_executor.kernels.linear",
                   _POSSIBLE_MXFP4_KERNELS={ROCM: [_OtherKernel], "cuda": [_OtherKernel]})
    mod("vllm.model_executor.kernels.linear.mxfp4")
    mod("vllm.model_executor.kernels.linear.mxfp4.base", MxFp4LinearKernel=MxFp4LinearKernel,
        MxFp4LinearLayerConfig=MxFp4LinearLayerConfig)
    mod("vllm.model_executor.layers")
    mod("vllm.model_executor.layers.quantization")
    mod("vllm.model_executor.layers.quantization.utils")
    mod("vllm.model_executor.layers.quantization.utils.quant_utils",
        kMxfp4Dynamic=K_MXFP4_DYNAMIC)
    for name, m in mods.items():
        monkeypatch.setitem(sys.modules, name, m)
    monkeypatch.setattr(R, "_KERNEL_CLS", None)
    yield types.SimpleNamespace(registry=registry, config=MxFp4LinearLayerConfig,
                                base=MxFp4LinearKernel, asm=asm)
    R._KERNEL_CLS = None          # the next kernel_class() call rebuilds on whatever is importable


def test_class_builds_on_vllm_abc(fake_vllm):
    cls = R.kernel_class()
    assert issubclass(cls, fake_vllm.base)
    assert cls.__name__ == "RadianceMxfp4W4A8LinearKernel"
    for name in ("is_supported", "can_implement", "process_weights_after_loading",
                 "apply_weights", "apply"):
        assert callable(getattr(cls, name)), name


def test_register_inserts_at_head_exactly_once(fake_vllm):
    reg = fake_vllm.registry._POSSIBLE_MXFP4_KERNELS
    assert R.register_with_vllm() is True
    cls = R.kernel_class()
    assert reg[ROCM] == [cls, _OtherKernel]
    assert R.register_with_vllm() is True           # idempotent: still once, still first
    assert reg[ROCM] == [cls, _OtherKernel]
    assert reg["cuda"] == [_OtherKernel]            # other platforms untouched


def test_register_moves_a_stale_entry_to_the_head(fake_vllm):
    reg = fake_vllm.registry._POSSIBLE_MXFP4_KERNELS
    cls = R.kernel_class()
    reg[ROCM].append(cls)
    R.register_with_vllm()
    assert reg[ROCM] == [cls, _OtherKernel]


def test_register_on_an_explicit_platform_key(fake_vllm):
    reg = fake_vllm.registry._POSSIBLE_MXFP4_KERNELS
    R.register_with_vllm("rocm-test")
    assert reg["rocm-test"] == [R.kernel_class()]


def test_register_without_vllm_returns_false(monkeypatch):
    monkeypatch.setitem(sys.modules, "vllm", None)   # import vllm... raises ImportError
    assert R.register_with_vllm() is False


def test_is_supported_declines_without_the_switch(fake_vllm, monkeypatch):
    monkeypatch.setattr(R, "ENABLED", False)
    ok, why = R.kernel_class().is_supported()
    assert ok is False and "RADIANCE_MXFP4_W4A8" in why


def test_is_supported_declines_when_the_library_is_missing(fake_vllm, monkeypatch):
    monkeypatch.setattr(R, "ENABLED", True)

    def missing():
        raise RuntimeError("libw4a8_mxfp4.so is not built")
    monkeypatch.setattr(_native, "lib", missing)
    ok, why = R.kernel_class().is_supported()
    assert ok is False and "failed to load" in why


def test_is_supported_declines_off_gfx950(fake_vllm, monkeypatch):
    monkeypatch.setattr(R, "ENABLED", True)
    monkeypatch.setattr(_native, "lib", lambda: object())
    monkeypatch.setattr(R, "on_gfx950", lambda: False)
    ok, why = R.kernel_class().is_supported()
    assert ok is False and "gfx950" in why


def test_is_supported_accepts_gfx950_with_switch_and_library(fake_vllm, monkeypatch):
    monkeypatch.setattr(R, "ENABLED", True)
    monkeypatch.setattr(_native, "lib", lambda: object())
    monkeypatch.setattr(R, "on_gfx950", lambda: True)
    assert R.kernel_class().is_supported() == (True, None)


def test_on_gfx950_is_false_without_a_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert R.on_gfx950() is False


def test_can_implement_requires_mxfp4_dynamic(fake_vllm):
    cls = R.kernel_class()
    assert cls.can_implement(fake_vllm.config(K_MXFP4_DYNAMIC)) == (True, None)
    ok, why = cls.can_implement(fake_vllm.config(K_OTHER))
    assert ok is False and "MXFP4 dynamic" in why


def test_can_implement_declines_aiter_asm_layout(fake_vllm):
    fake_vllm.asm.enabled = True
    ok, why = R.kernel_class().can_implement(fake_vllm.config(K_MXFP4_DYNAMIC))
    assert ok is False and "AITER" in why


def _install_backend_filter(fake_vllm, monkeypatch, keep):
    """A stand-in for vLLM's --linear-backend filter (_resolve_backend_kernels): with a backend
    set, only the kernels it names survive; and init_mxfp4_linear_kernel's order of operations
    (list, filter, first kernel whose is_supported and can_implement accept)."""
    registry = fake_vllm.registry

    def _resolve_backend_kernels(possible, quantization):
        return [k for k in possible if k in keep]
    monkeypatch.setattr(registry, "_resolve_backend_kernels", _resolve_backend_kernels,
                        raising=False)

    def init_mxfp4_linear_kernel(cfg):
        possible = list(registry._POSSIBLE_MXFP4_KERNELS.get(ROCM, []))
        possible = registry._resolve_backend_kernels(possible, "MXFP4")
        for k in possible:
            if k is _OtherKernel:
                return k, possible
            if k.is_supported()[0] and k.can_implement(cfg)[0]:
                return k, possible
        return None, possible
    return init_mxfp4_linear_kernel


def test_registration_survives_the_linear_backend_filter(fake_vllm, monkeypatch):
    """With --linear-backend naming another kernel, the filter drops every class it does not name;
    the reference's insertion point (after the filter, sly/patch_quark_mxfp4.py:74-103) keeps the
    plugin at the head anyway, and so does register_with_vllm."""
    monkeypatch.setattr(_native, "lib", lambda: object())
    monkeypatch.setattr(R, "on_gfx950", lambda: True)
    monkeypatch.setattr(R, "ENABLED", True)
    init = _install_backend_filter(fake_vllm, monkeypatch, keep={_OtherKernel})
    cfg = fake_vllm.config(K_MXFP4_DYNAMIC)
    assert init(cfg)[0] is _OtherKernel                  # not registered: the backend's kernel
    R.register_with_vllm()
    R.register_with_vllm()                               # idempotent: the filter wrapped once
    picked, possible = init(cfg)
    assert picked is R.kernel_class()
    assert possible == [R.kernel_class(), _OtherKernel]
    # other quantizations and an unfiltered list pass through unchanged
    resolve = fake_vllm.registry._resolve_backend_kernels
    assert resolve([R.kernel_class(), _OtherKernel], "FP8") == [_OtherKernel]
    assert resolve([_OtherKernel], quantization="mxfp4") == [_OtherKernel]
    monkeypatch.setattr(R, "ENABLED", False)             # declining still hands the layer on
    assert init(cfg)[0] is _OtherKernel


def test_selection_order_picks_the_plugin_first(fake_vllm, monkeypatch):
    """What init_mxfp4_linear_kernel does with the list: the first class whose is_supported and
    can_implement both accept. With the plugin registered and accepting it is chosen; declining
    (switch off) hands the layer to the next kernel."""
    monkeypatch.setattr(_native, "lib", lambda: object())
    monkeypatch.setattr(R, "on_gfx950", lambda: True)
    R.register_with_vllm()
    cfg = fake_vllm.config(K_MXFP4_DYNAMIC)

    def select():
        for k in fake_vllm.registry._POSSIBLE_MXFP4_KERNELS[ROCM]:
            if k is _OtherKernel:
                return k
            if k.is_supported()[0] and k.can_implement(cfg)[0]:
                return k
        return None

    monkeypatch.setattr(R, "ENABLED", True)
    assert select() is R.kernel_class()
    monkeypatch.setattr(R, "ENABLED", False)
    assert select() is _OtherKernel
