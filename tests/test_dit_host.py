"""CPU checks of the synthetic DiT stack harness: which linears the Flux 2
skip list leaves to the quantizer (on the meta-device skeleton the loader
builds for LoRA key discovery), the LoRA patch map, the work count, and one
small forward of the stack with plain bf16 linears."""
import pytest
import torch

import dit_stack as ds
from conftest import import_pkg
from fake_comfy import FakeLoRA, install_fake_comfy


@pytest.fixture(scope="module")
def Ops():
    install_fake_comfy()
    from importlib import import_module, reload
    import_pkg()
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = reload(m)
    return m.Int4ConvRotOps


def test_skip_list_selects_block_linears(Ops):
    saved = (Ops.skeleton_meta_init, list(Ops.excluded_names), Ops.min_in_features)
    Ops.skeleton_meta_init = True
    Ops.excluded_names = list(ds.FLUX2_EXCLUDED)
    Ops.min_in_features = 512
    try:
        model = ds.DoubleStreamDiT(Ops, depth=3)
        chosen = {n for n, m in model.named_modules()
                  if hasattr(m, "in_features") and m._should_quantize(n + ".", m.weight)}
    finally:
        Ops.skeleton_meta_init, Ops.excluded_names, Ops.min_in_features = saved
    want = {f"double_blocks.{i}.{s}" for i in range(3) for s in ds.QUANTIZED_SUFFIXES}
    assert chosen == want
    shapes = ds.linear_shapes(model)
    # the excluded linears wide enough to be quantized without the skip list
    assert shapes["txt_in"] == (4096, 3072) and shapes["double_stream_modulation_img.lin"] == (3072, 18432)
    assert shapes["double_blocks.2.img_mlp.2"] == (12288, 3072)


def test_lora_patch_map_covers_quantized_linears():
    install_fake_comfy()
    import comfy.ops
    model = ds.DoubleStreamDiT(comfy.ops.manual_cast, depth=2, hidden=256, heads=4, context_dim=64)
    patches = ds.lora_patches_for(model, FakeLoRA, rank=32)
    assert set(patches) == {f"double_blocks.{i}.{s}.weight" for i in range(2) for s in ds.QUANTIZED_SUFFIXES}
    v = patches["double_blocks.1.img_mlp.0.weight"][0][0]
    up, down, alpha = v.weights[:3]
    assert up.shape == (1024, 32) and down.shape == (32, 256) and alpha == 32.0


def test_quantized_work_count():
    # 8 blocks x 2 streams x (qkv + proj + mlp_up + mlp_down) at 4096 + 512 tokens
    assert ds.quantized_work(4096, 512) == 8 * 2 * 4608 * 3072 * (9216 + 3072 + 12288 + 12288)
    assert ds.quantized_work(4096, 512, lora_rank=32) - ds.quantized_work(4096, 512) == \
        8 * 2 * 4608 * 32 * ((3072 + 9216) + (3072 + 3072) + (3072 + 12288) + (12288 + 3072))


def test_small_stack_forward_bf16():
    install_fake_comfy()
    import comfy.ops
    model = ds.DoubleStreamDiT(comfy.ops.manual_cast, depth=2, hidden=256, heads=4, context_dim=64)
    model.load_state_dict(ds.state_dict_for(model, seed=3), strict=True)
    img, ctx, t = ds.synthetic_inputs(12, 5, context_dim=64)
    with torch.no_grad():
        y = model(img, ctx, t)
        y2 = model(img, ctx, t)
    assert y.shape == (1, 12, 64) and y.dtype == torch.bfloat16
    assert torch.isfinite(y.float()).all() and torch.equal(y, y2)


def test_attention_matches_closed_form():
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn((1, 6, 9, 16), generator=g).to(torch.bfloat16) for _ in range(3))
    got = ds.attention(q, k, v, head_chunk=4).float()
    qf, kf, vf = q.double(), k.double(), v.double()
    p = torch.softmax(qf @ kf.transpose(-1, -2) / 4.0, dim=-1)
    want = (p @ vf).permute(0, 2, 1, 3).reshape(1, 9, 96)
    assert float((got.double() - want).abs().max()) < 0.03
