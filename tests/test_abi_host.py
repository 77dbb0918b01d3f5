"""CPU-only checks: the C-ABI library loads and exports what the header
declares, the host-side API validates like the reference, the codec and the
Linear replacement's load-time dispatch logic (with a fake comfy package)."""
import ctypes
import importlib
import os
import re
import sys
import types

import numpy as np
import pytest
import torch

from conftest import ROOT, import_pkg
from fake_comfy import install_fake_comfy


def header_symbols():
    text = open(os.path.join(ROOT, "include", "convrot_mi355x.h")).read()
    return re.findall(r"^\s*(?:int|size_t)\s+(\w+)\s*\(", text, flags=re.M)


def test_header_declares_reference_entry_points():
    syms = header_symbols()
    # names a binding of the reference's ctypes loader resolves (hip_loader.py:50-61)
    assert "ck_convrot_quant_int4" in syms
    assert "ck_int4_convrot_gemm" in syms
    # the int8 tier's pair (hip_loader.py:63-71)
    assert "ck_convrot_quant_int8" in syms
    assert "ck_int8_convrot_gemm" in syms


def test_library_exports_every_declared_symbol(native):
    lib = native.load_library()
    for name in header_symbols():
        assert hasattr(lib, name), name
    raw = ctypes.CDLL(native.lib_path())
    for name in header_symbols():
        getattr(raw, name)
    assert set(native.exported_symbols()) == set(header_symbols())


# What the reference's ctypes loader binds, name by name, with the argtypes it
# installs (reference _int4/hip_loader.py:50-71): pointers (c_void_p) and ints.
REFERENCE_BINDINGS = {
    "ck_int4_convrot_gemm": [ctypes.c_void_p] * 6 + [ctypes.c_int] * 4 + [ctypes.c_void_p],
    "ck_int4_convrot_gemm_splitk": [ctypes.c_void_p] * 5 + [ctypes.c_int] * 4 + [ctypes.c_void_p],
    "ck_convrot_quant_int4": [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                              ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p],
    "ck_int8_convrot_gemm": [ctypes.c_void_p] * 6 + [ctypes.c_int] * 4 + [ctypes.c_void_p],
    "ck_convrot_quant_int8": [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                              ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p],
}


def test_reference_loader_binds_this_library(native):
    """The reference loader's _ensure_loaded resolves all five symbols
    unconditionally; each must exist with an int return and the same argument
    list as in the header (same count and kinds), and reject bad arguments
    with -1 exactly as the reference does, before touching the device."""
    lib = ctypes.CDLL(native.lib_path())
    text = open(os.path.join(ROOT, "include", "convrot_mi355x.h")).read()
    for name, argtypes in REFERENCE_BINDINGS.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = argtypes
        decl = re.search(r"^int\s+" + name + r"\s*\(([^;]*)\);", text, flags=re.M | re.S)
        assert decl, name
        params = [a.strip() for a in decl.group(1).split(",")]
        assert len(params) == len(argtypes), name
        for p, t in zip(params, argtypes):
            assert ("*" in p) == (t is ctypes.c_void_p), (name, p)
    n = None
    assert lib.ck_int4_convrot_gemm(n, n, n, n, n, n, 4, 4, 48, 1, n) == -1          # K % 32
    assert lib.ck_int4_convrot_gemm_splitk(n, n, n, n, n, 4, 4, 48, 2, n) == -1     # K % 32
    assert lib.ck_int4_convrot_gemm_splitk(n, n, n, n, n, 4, 4, 64, 0, n) == -1     # nsplit < 1
    assert lib.ck_int4_convrot_gemm_splitk(n, n, n, n, n, 0, 4, 64, 2, n) == 0      # empty: nothing to do
    assert lib.ck_convrot_quant_int4(n, 1, n, n, 4, 256, 32, n) == -1              # G not 16/64/256
    assert lib.ck_int8_convrot_gemm(n, n, n, n, n, n, 4, 4, 40, 1, n) == -1          # K % 16
    assert lib.ck_convrot_quant_int8(n, 1, n, n, 4, 100, 16, n) == -1              # K % G


def test_load_refuses_other_abi_version(native, monkeypatch):
    """Bindings for another ABI version refuse the library instead of calling
    it with mismatched arguments."""
    monkeypatch.setattr(native, "_lib", None)
    monkeypatch.setattr(native, "ABI_VERSION", native.ABI_VERSION + 1)
    with pytest.raises(RuntimeError, match="ABI version"):
        native.load_library()


def test_library_queries_without_gpu(native):
    lib = native.load_library()
    assert lib.cr_abi_version() == native.ABI_VERSION == 13
    assert lib.cr_max_quant_k() == 32768
    assert lib.cr_max_quant_bf6_k() == 32768


def test_argument_errors_return_minus_one(native):
    """Invalid arguments are rejected before any device work (-1)."""
    lib = native.load_library()
    n = ctypes.c_void_p(0)
    assert lib.ck_convrot_quant_int4(n, 1, n, n, 4, 256, 32, n) == -1      # bad G
    assert lib.ck_convrot_quant_int4(n, 1, n, n, 4, 100, 16, n) == -1      # K % G
    assert lib.ck_convrot_quant_int4(n, 7, n, n, 4, 256, 256, n) == -1     # bad dtype
    assert lib.ck_convrot_quant_int4(n, 1, n, n, 4, 65536, 256, n) == -1   # K too large
    assert lib.ck_int4_convrot_gemm(n, n, n, n, n, n, 4, 4, 48, 1, n) == -1  # K % 32
    assert lib.ck_int4_convrot_gemm(n, n, n, n, n, n, 4, 4, 64, 5, n) == -1  # out dtype
    assert lib.cr_int4_convrot_gemm_ex(n, n, n, n, n, n, 4, 4, 64, 9, n) == -1
    assert lib.cr_convrot_quant_int4_stochastic(n, 1, n, n, n, 4, 256, 256, n) == -1  # no noise
    f = ctypes.c_float(1.0)
    assert lib.cr_lora_down(n, 1, n, n, 4, 256, 48, n, 0, n) == -1        # rank not a multiple of 32
    assert lib.cr_lora_down(n, 1, n, n, 4, 256, 160, n, 0, n) == -1       # rank above 128
    assert lib.cr_lora_down(n, 0, n, n, 4, 256, 32, n, 0, n) == -1        # f32 input
    assert lib.cr_lora_down(n, 1, n, n, 4, 40, 32, n, 0, n) == -1         # K % 16
    assert lib.cr_lora_down(n, 1, n, n, 4, 512, 32, n, 0, n) == -1        # split shape, no workspace
    # the split plan, a function of the shape only: 64-row workgroups over 4 k
    # ranges for the image stream's long rows, 16-row ones over the whole of K
    # for its short rows (no partials), 16-row ones over 8 ranges for the text stream
    # the split counter region (2 KB) leads every workspace
    assert lib.cr_lora_down_workspace(4096, 12288, 32) == 2048 + 4 * 4096 * 32 * 4
    assert lib.cr_lora_down_workspace(4096, 3072, 32) == 0
    assert lib.cr_lora_down_workspace(512, 3072, 32) == 2048 + 8 * 512 * 32 * 4
    assert lib.cr_lora_down_workspace(4608, 3072, 64) == 2048 + 4 * 4608 * 64 * 4
    assert lib.cr_lora_down_workspace(64, 256, 32) == 0                    # K of one 256-k range: one split
    assert lib.cr_lora_down_workspace(4, 40, 32) == 0
    assert lib.cr_int4_convrot_gemm_lora(n, n, n, n, n, n, n, 32, f, n, 4, 4, 64, 3, n) == -1  # acc dump
    assert lib.cr_int4_convrot_gemm_lora(n, n, n, n, n, n, n, 32, f, n, 4, 4, 64, 0, n) == -1  # null t/U
    assert lib.cr_int4_convrot_gemm_lora(n, n, n, n, n, n, n, 64, f, n, 4, 4, 48, 0, n) == -1  # K % 32
    assert lib.cr_convrot_quant_bf6(n, 1, n, n, 4, 192, 64, n) == -1          # K % 128
    assert lib.cr_convrot_quant_bf6(n, 1, n, n, 4, 33024, 256, n) == -1       # above the bf6 quantizer's K
    assert lib.cr_int4_to_bf6(n, n, 4, 96, n) == -1                           # K % 128
    assert lib.cr_bf6_to_int4(n, n, 4, 96, n) == -1                           # K % 128
    assert lib.cr_int4_convrot_gemm_bf6(n, n, n, n, n, n, 4, 4, 192, 0, n) == -1
    assert lib.cr_int4_convrot_gemm_bf6(n, n, n, n, n, n, 4, 4, 256, 4, n) == -1
    assert lib.ck_convrot_quant_int8(n, 1, n, n, 4, 256, 32, n) == -1      # bad G
    assert lib.ck_convrot_quant_int8(n, 1, n, n, 4, 100, 16, n) == -1      # K % G
    assert lib.ck_convrot_quant_int8(n, 3, n, n, 4, 256, 256, n) == -1     # bad dtype
    assert lib.ck_int8_convrot_gemm(n, n, n, n, n, n, 4, 4, 40, 1, n) == -1  # K % 16
    assert lib.ck_int8_convrot_gemm(n, n, n, n, n, n, 4, 4, 64, 2, n) == -1  # out dtype
    assert lib.cr_int8_convrot_gemm_ex(n, n, n, n, n, n, 4, 4, 64, 2, n) == -1  # no eager bf16 chain for int8
    assert lib.cr_convrot_quant_int8_i8t(n, 1, n, n, 4, 160, 16, n) == -1      # K % 64
    assert lib.cr_convrot_quant_int8_i8t(n, 1, n, n, 4, 33024, 256, n) == -1   # above the row quantizer's K
    assert lib.cr_int8_to_i8t(n, n, 4, 96, n) == -1                             # K % 64
    assert lib.cr_i8t_to_int8(n, n, 4, 96, n) == -1                             # K % 64
    assert lib.cr_int8_to_i8t(n, n, -1, 64, n) == -1                            # rows < 0
    assert lib.cr_int8_convrot_gemm_i8t(n, n, n, n, n, n, 4, 4, 96, 1, n) == -1  # K % 64
    assert lib.cr_int8_convrot_gemm_i8t(n, n, n, n, n, n, 4, 4, 64, 2, n) == -1  # no eager bf16 chain
    sk = lib.cr_int4_convrot_gemm_bf6_splitk
    assert sk(n, n, n, n, n, n, n, 0, f, n, 4, 4, 256, 0, 0, n, 0, n) == -1        # nsplit < 1
    assert sk(n, n, n, n, n, n, n, 0, f, n, 4, 4, 256, 0, 3, n, 1 << 30, n) == -1  # more splits than 128-k blocks
    assert sk(n, n, n, n, n, n, n, 0, f, n, 4, 4, 256, 0, 2, n, 1 << 30, n) == -1  # no workspace
    ws_need = lib.cr_gemm_bf6_splitk_workspace(4, 4, 2)
    assert sk(n, n, n, n, n, n, n, 0, f, n, 4, 4, 256, 0, 2, ctypes.c_void_p(16), ws_need - 1, n) == -1
    assert sk(n, n, n, n, n, ctypes.c_void_p(16), n, 32, f, n, 4, 4, 256, 3, 1, n, 0, n) == -1  # acc dump with LoRA


def test_pick_groupsize(backend):
    assert backend.pick_groupsize(3072) == 256
    assert backend.pick_groupsize(12288) == 256
    assert backend.pick_groupsize(3840) == 256
    assert backend.pick_groupsize(192) == 64
    assert backend.pick_groupsize(80) == 16
    assert backend.pick_groupsize(40) is None


def test_linear_validation_errors(backend):
    x = torch.zeros(4, 512, dtype=torch.bfloat16)
    qw = torch.zeros(8, 256, dtype=torch.int8)
    ws = torch.ones(8)
    with pytest.raises(ValueError):
        backend.convrot_w4a4_linear(x, qw, ws, linear_dtype="fp8")
    with pytest.raises(ValueError):
        backend.convrot_w4a4_linear(x, qw, ws, quant_group_size=32)
    with pytest.raises(ValueError):
        backend.convrot_w4a4_linear(x, torch.zeros(8, 128, dtype=torch.int8), ws)
    with pytest.raises(ValueError):
        backend.convrot_w4a4_linear(torch.zeros(4, 80, dtype=torch.bfloat16),
                                    torch.zeros(8, 40, dtype=torch.int8), ws, convrot_groupsize=256)
    qw = torch.zeros(8, 256, dtype=torch.int8)
    with pytest.raises(ValueError, match="wscales"):                 # N scales
        backend.convrot_w4a4_linear(x, qw, torch.ones(7))
    with pytest.raises(ValueError, match="bias"):                    # N biases
        backend.convrot_w4a4_linear(x, qw, ws, bias=torch.zeros(9))
    D = torch.zeros(32, 512, dtype=torch.bfloat16)
    U = torch.zeros(8, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="bf16"):                    # LoRA dtype
        backend.convrot_w4a4_linear(x, qw, ws, lora=(D.half(), U))
    with pytest.raises(ValueError, match="contiguous"):              # LoRA layout
        backend.convrot_w4a4_linear(x, qw, ws, lora=(D, torch.zeros(32, 8, dtype=torch.bfloat16).T))
    with pytest.raises(ValueError, match="LoRA shapes"):
        backend.convrot_w4a4_linear(x, qw, ws, lora=(D, torch.zeros(8, 64, dtype=torch.bfloat16)))


def test_weight_validation_errors(backend):
    with pytest.raises(ValueError):
        backend.quantize_convrot_w4a4_weight(torch.zeros(8, 512), quant_group_size=32)
    with pytest.raises(ValueError):
        backend.quantize_convrot_w4a4_weight(torch.zeros(8, 80), convrot_groupsize=16)  # K % 64
    with pytest.raises(ValueError):
        backend.quantize_convrot_w4a4_weight(torch.zeros(8, 8, 8))


def test_codec_torch_roundtrip(backend, oracle):
    from importlib import import_module
    codec = import_module("comfyui-int4-convrot-rdna4_amd._int4._codec")
    allb = torch.arange(-128, 128, dtype=torch.int32).to(torch.int8).reshape(2, 128)
    codes = codec._unpack_int4_row_major(allb)
    assert np.array_equal(codes.numpy(), oracle.unpack(allb.numpy()))
    assert torch.equal(codec._pack_int4_row_major(codes), allb)
    assert codec._INT4_GROUP_SIZE == 64 and codec._INT4_MAX == 7


def test_dequantize_matches_oracle(backend, oracle, goldens):
    q = torch.from_numpy(goldens["w64_q"])
    s = torch.from_numpy(goldens["w64_s"])
    deq = backend.dequantize_convrot_w4a4_weight(q, s, convrot_groupsize=64)
    np.testing.assert_allclose(deq.numpy(), goldens["w64_deq"], rtol=0, atol=2e-6)


# ----------------------------------------------------------------------------
# Int4ConvRotOps load-time logic with a fake comfy package
# ----------------------------------------------------------------------------

@pytest.fixture(scope="module")
def ops_mod():
    install_fake_comfy()
    from importlib import import_module, reload
    import_pkg()
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = reload(m)
    assert m.Int4ConvRotOps is not None
    return m


def test_ops_should_quantize_and_mode(ops_mod):
    Ops = ops_mod.Int4ConvRotOps
    Ops.excluded_names = ["img_in"]
    Ops.excluded_exact = {"double_blocks.0.img_attn.proj"}
    Ops.int8_exact = {"double_blocks.0.img_mlp.0"}
    try:
        lin = Ops.Linear(3072, 64, bias=True)
        w = torch.zeros(64, 3072)
        assert lin._should_quantize("diffusion_model.double_blocks.0.img_attn.qkv.", w)
        assert not lin._should_quantize("diffusion_model.img_in.", w)
        assert not lin._should_quantize("diffusion_model.double_blocks.0.img_attn.proj.", w)
        assert lin._quant_mode("model.diffusion_model.double_blocks.0.img_mlp.0.") == "int8"
        assert lin._quant_mode("double_blocks.0.img_mlp.2.") == "int4"
        small = Ops.Linear(256, 64)
        assert not small._should_quantize("x.", torch.zeros(64, 256))      # < min_in_features
        odd = Ops.Linear(520, 64)
        assert not odd._should_quantize("x.", torch.zeros(64, 520))        # no groupsize
        assert not lin._should_quantize("x.", torch.zeros(3072))           # not 2-D
    finally:
        Ops.excluded_names, Ops.excluded_exact, Ops.int8_exact = [], set(), set()


def test_ops_key_normalization(ops_mod):
    L = ops_mod.Int4ConvRotOps.Linear
    assert L._normalize_lora_key("diffusion_model.a.b.weight") == "a.b.weight"
    assert L._normalize_lora_key("transformer.x") == "x"
    assert L._exact_key("model.diffusion_model.blk.0.") == "blk.0"
    assert L._normalize_lora_key(3) == 3


def test_ops_quant_tag_parsing(ops_mod):
    tag = lambda d: torch.tensor(list(__import__("json").dumps(d).encode()), dtype=torch.uint8)
    assert ops_mod._parse_quant_tag(tag({"format": "convrot_w4a4", "convrot_groupsize": 64})) == (True, 64)
    assert ops_mod._parse_quant_tag(tag({"format": "float8_e4m3fn"})) == (False, None)
    assert ops_mod._parse_quant_tag(tag({"format": "int8_tensorwise"})) == (False, None)
    assert ops_mod._parse_quant_tag(tag({"format": "int8_tensorwise", "convrot": True})) == (True, None)


def test_ops_plain_layer_loads_bf16(ops_mod):
    """A layer that is not quantized (too narrow) takes the plain load path."""
    lin = ops_mod.Int4ConvRotOps.Linear(256, 32, bias=True)
    sd = {"weight": torch.randn(32, 256), "bias": torch.randn(32)}
    lin.load_state_dict(sd)
    assert lin._q is None and lin._qmode is None
    x = torch.randn(3, 256)
    torch.testing.assert_close(lin(x), x @ sd["weight"].T + sd["bias"])


def test_ops_refuses_unknown_prequant_layout(ops_mod):
    lin = ops_mod.Int4ConvRotOps.Linear(3072, 32, bias=False)
    sd = {"weight": torch.zeros(32, 100, dtype=torch.int8), "weight_scale": torch.ones(32)}
    assert lin._load_prequantized(dict(sd), "", "weight", "weight_scale", sd["weight"]) is False


def test_split_choice_and_workspace(native):
    """The k-split choice is host arithmetic: large tile grids never split,
    small-M / large-K products do, within 2 .. nkb; the workspace is the 2 KB
    counter region plus one f32 per output of every tile and split of the
    largest tile shape (here the 256 x 256 one's S * tiles * 256 KB)."""
    lib = native.load_library()
    assert lib.cr_gemm_bf6_choose_nsplit(4608, 3072, 3072) == 1
    assert lib.cr_gemm_bf6_choose_nsplit(4608, 12288, 3072) == 1
    s = lib.cr_gemm_bf6_choose_nsplit(512, 3072, 12288)
    assert 2 <= s <= 96
    assert lib.cr_gemm_bf6_choose_nsplit(256, 256, 256) <= 2
    assert lib.cr_gemm_bf6_splitk_workspace(512, 3072, 4) == 2048 + 4 * 24 * 256 * 256 * 4
    assert lib.cr_gemm_bf6_splitk_workspace(300, 300, 2) == 2048 + 2 * 4 * 256 * 256 * 4
    assert lib.cr_gemm_bf6_splitk_workspace(300, 300, 1) == 0


def test_tile_choice(native):
    """The workgroup tile and the split count are host arithmetic: 256 x 256
    on large grids; on small grids 128 x 192 exactly when 128 x 128 tiles
    (times the splits) exceed the 256 CUs and 128 x 192 tiles do not; bad
    arguments are refused."""
    tile = native.gemm_tile_bf6
    assert tile(4608, 3072, 3072) == (256, 256)
    assert tile(512, 3072, 3072) == (128, 128)                # 96 quarter tiles
    assert tile(1024, 3072, 3072) == (128, 128)               # 192
    assert tile(512, 9216, 3072) == (128, 192)                # 288 -> 192
    assert tile(512, 12288, 3072) == (128, 192)               # 384 -> 256
    assert tile(2048, 3072, 3072) == (128, 192)               # 384 -> 256
    assert tile(512, 15360, 3840) == (128, 128)               # 480 -> 320: both exceed the CUs
    assert tile(768, 9216, 3072) == (128, 128)                # 432 -> 288
    assert tile(9000, 449, 1024) == (128, 192)                # 284 -> 213, ragged, edge units clamped
    assert tile(512, 12288, 3072, nsplit=2) == (128, 128)     # 768 split workgroups -> 512: neither fits
    assert tile(512, 3072, 12288, nsplit=2) == (128, 128)     # 192 split workgroups
    assert native.choose_nsplit_bf6(512, 3072, 12288) == 2
    assert native.choose_nsplit_bf6(1024, 3072, 12288) == 2   # 192 quarter tiles, long rows:
    assert tile(1024, 3072, 12288, nsplit=2) == (128, 192)    # 384 split workgroups -> 256
    assert native.choose_nsplit_bf6(768, 3072, 12288) == 2
    assert tile(768, 3072, 12288, nsplit=2) == (128, 192)
    assert native.choose_nsplit_bf6(1024, 3072, 6144) == 1    # 48 blocks: a split of 192 tiles does not pay
    assert native.choose_nsplit_bf6(256, 3072, 12288) == 4
    assert tile(256, 3072, 12288, nsplit=4) == (128, 128)
    lib = native.load_library()
    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    for args in [(0, 1, 128, 1), (1, 1, 100, 1), (1, 1, 128, 2), (1, 1, 128, 0)]:
        assert lib.cr_gemm_bf6_tile(*args, ctypes.byref(bm), ctypes.byref(bn)) == -1, args
    assert lib.cr_gemm_bf6_tile(1, 1, 128, 1, None, None) == -1


def test_ops_meta_skeleton(ops_mod):
    """skeleton_meta_init builds meta-device parameters (the loader's LoRA
    key-map discovery pass) with the quantized-state attributes unset."""
    Ops = ops_mod.Int4ConvRotOps
    Ops.skeleton_meta_init = True
    try:
        a = Ops.Linear(3072, 64, bias=True, dtype=torch.bfloat16)
        b = Ops.Linear(3072, 64, bias=False)
    finally:
        Ops.skeleton_meta_init = False
    assert a.weight.device.type == "meta" and a.weight.shape == (64, 3072) and a.weight.dtype == torch.bfloat16
    assert a.bias.device.type == "meta" and a.bias.shape == (64,)
    assert b.bias is None and b.weight.device.type == "meta"
    for m in (a, b):
        assert m._q is None and m._qs is None and m._qgs is None and m._qmode is None and m._dyn_lora is None
        assert m.in_features == 3072 and m.out_features == 64


def test_ops_lora_routing_without_quantization(ops_mod):
    """A layer that stays bf16 folds its LoRA patches into weight and bias
    (through comfy.lora.calculate_weight) even in dynamic mode; patches of
    adapters without an additive bypass are refused for the side path."""
    import comfy
    calls = []

    def calculate_weight(patches, t, key):
        calls.append((key, [p[0] for p in patches]))
        return t + 1.0
    comfy.lora = types.SimpleNamespace(calculate_weight=calculate_weight)
    comfy.model_management = types.SimpleNamespace(lora_compute_dtype=lambda dev: torch.float32)
    sys.modules["comfy.lora"], sys.modules["comfy.model_management"] = comfy.lora, comfy.model_management
    Ops = ops_mod.Int4ConvRotOps
    Ops.lora_patches = {"blk.lin.weight": [("patch", None, None, 0.5)], "blk.lin.bias": [("patch", None, None)]}
    Ops.lora_dynamic = True
    try:
        lin = Ops.Linear(256, 32, bias=True)                  # narrower than min_in_features: stays bf16
        sd = {"diffusion_model.blk.lin.weight": torch.zeros(32, 256), "diffusion_model.blk.lin.bias": torch.zeros(32)}
        lin._load_from_state_dict(sd, "diffusion_model.blk.lin.", {}, True, [], [], [])
        assert lin._q is None and lin._dyn_lora is None
        assert torch.equal(lin.weight, torch.ones(32, 256)) and torch.equal(lin.bias, torch.ones(32))
        assert calls == [("diffusion_model.blk.lin.weight", [0.5]), ("diffusion_model.blk.lin.bias", [1.0])]
        assert Ops._applied_lora == {"blk.lin.weight", "blk.lin.bias"}
        assert lin._prepare_dyn_adapters([("raw diff tensor", None, None, 1.0)]) is None
    finally:
        Ops.lora_patches, Ops.lora_dynamic, Ops._applied_lora = {}, False, set()
        for k in ("comfy.lora", "comfy.model_management"):
            sys.modules.pop(k, None)


def test_workspace_cache_reuses_grows_and_is_bounded(monkeypatch):
    """The Python layer's per-stream workspace: reused by later calls on the
    same stream, replaced when a call needs more, one per stream, and at most
    _MAX_WORKSPACES streams kept (least recently used dropped first)."""
    import importlib
    from conftest import PKG_NAME
    import_pkg()
    native = importlib.import_module(PKG_NAME + "._int4.native")
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: False)
    monkeypatch.setattr(native, "_workspaces", type(native._workspaces)())
    dev = torch.device("cpu")
    a = native._workspace(dev, 1, 3000)
    assert int(a[:native.SPLIT_COUNTER_BYTES].count_nonzero()) == 0      # split counters start at zero
    assert native._workspace(dev, 1, 50) is a
    b = native._workspace(dev, 1, 5000)
    assert b is not a and b.numel() >= 5000
    assert native._workspace(dev, 2, 10) is not b
    for s in range(3, 3 + native._MAX_WORKSPACES):
        native._workspace(dev, s, 10)
    assert len(native._workspaces) == native._MAX_WORKSPACES
    assert (None, 1) not in native._workspaces and (None, 2) not in native._workspaces
    assert (None, 2 + native._MAX_WORKSPACES) in native._workspaces


def test_too_wide_rows_stay_bf16(ops_mod, backend):
    """in_features above the fused quantizer's 32768: the API raises a
    ValueError with the reason before any device work, a float layer is not
    quantized (logged), and a prequantized int4 or int8 layer loads dequantized
    in bf16 from its stored codes (the reference rotates such rows with torch,
    _int4/__init__.py:59-66)."""
    import logging
    K = 33024                                      # 129 groups of 256
    assert backend.max_quant_k() == 32768
    with pytest.raises(ValueError, match="exceeds 32768"):
        backend.quantize_convrot_w4a4_weight(torch.zeros(4, K))
    with pytest.raises(ValueError, match="exceeds 32768"):
        backend.convrot_w4a4_linear(torch.zeros(2, K), torch.zeros(4, K // 2, dtype=torch.int8), torch.ones(4))
    with pytest.raises(ValueError, match="exceeds 32768"):
        backend.convrot_w8a8_linear(torch.zeros(2, K), torch.zeros(4, K, dtype=torch.int8), torch.ones(4))
    Ops = ops_mod.Int4ConvRotOps
    lin = Ops.Linear(K, 4, bias=False)
    assert not lin._should_quantize("x.", torch.zeros(4, K))
    records = []
    handler = logging.Handler()
    handler.emit = records.append
    logging.getLogger().addHandler(handler)
    try:
        lin._load_from_state_dict({"x.weight": torch.ones(4, K, dtype=torch.bfloat16)}, "x.", {}, True, [], [], [])
        assert lin._qmode is None and bool((lin.weight == 1).all())      # a plain layer (the stand-in keeps f32)
        assert any("exceeds 32768" in r.getMessage() for r in records)
        g = torch.Generator().manual_seed(5)
        for mode, cols in (("int4", K // 2), ("int8", K)):
            q = torch.randint(-100, 100, (4, cols), generator=g, dtype=torch.int8)
            s = torch.rand(4, generator=g) * 0.01 + 0.001
            pre = Ops.Linear(K, 4, bias=False)
            pre._load_from_state_dict({"p.weight": q, "p.weight_scale": s}, "p.", {}, True, [], [], [])
            assert pre._qmode is None and pre._q is None, mode
            deq = (backend.dequantize_convrot_w4a4_weight(q, s, 256) if mode == "int4" else
                   importlib.import_module(backend.__name__ + ".int8_eager").dequantize_convrot_w8a8_weight(q, s, 256))
            assert torch.equal(pre.weight.data, deq.to(torch.bfloat16).to(pre.weight.dtype)), mode
        assert any("loading it dequantized" in r.getMessage() for r in records)
    finally:
        logging.getLogger().removeHandler(handler)


def test_split_workspace_covers_every_launch(native):
    """Host arithmetic the kernels' memory safety rests on, over random shapes
    and every split count a caller may pass: the workspace holds the counter
    region plus one f32 per output of every tile and split of the tile shape
    that launch runs, a split small-tile grid needs at most 512 counters, and
    the one-call linear's workspace holds its split partials, B6T codes,
    scales and t."""
    lib = native.load_library()
    rs = np.random.RandomState(11)
    bm, bn = ctypes.c_int(0), ctypes.c_int(0)
    for _ in range(400):
        M = int(rs.choice([1, 7, 64, 255, 256, 300, 512, 1000, 1024, 2048, 4608, 9000, 16384]) + rs.randint(0, 3))
        N = int(rs.choice([1, 64, 200, 449, 700, 3000, 3072, 9216, 12288, 13312]) + rs.randint(0, 3))
        K = 128 * int(rs.randint(1, 120))
        for ns in sorted({1, 2, 3, lib.cr_gemm_bf6_choose_nsplit(M, N, K), int(rs.randint(1, K // 128 + 1))}):
            if ns > K // 128:
                continue
            assert lib.cr_gemm_bf6_tile(M, N, K, ns, ctypes.byref(bm), ctypes.byref(bn)) == 0
            tiles = ((M + bm.value - 1) // bm.value) * ((N + bn.value - 1) // bn.value)
            ws = lib.cr_gemm_bf6_splitk_workspace(M, N, ns)
            if ns == 1:
                assert ws == 0
                continue
            assert ws >= 2048 + ns * tiles * bm.value * bn.value * 4, (M, N, K, ns, bm.value, bn.value)
            if bm.value == 128:
                assert tiles <= 512, (M, N, K, ns)
        for R in (0, 32):
            need = lib.cr_convrot_w4a4_linear_bf6_workspace(M, N, K, R)
            ns = lib.cr_gemm_bf6_choose_nsplit(M, N, K)
            rows = (M + 255) // 256 * 256
            floor = max(lib.cr_gemm_bf6_splitk_workspace(M, N, ns), 2048) + rows * K * 3 // 4 + 4 * M + 2 * M * R
            assert need >= floor, (M, N, K, R)
