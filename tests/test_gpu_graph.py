"""HIP-graph capture of the synthetic double-stream DiT stack's forward through
Int4ConvRotOps (every quantized linear one library call with its fused
rank-32 LoRA; attention, norms and the skip-list layers in torch): each
replay, with eager forwards of other token counts on the same library and
device synchronisations between the replays, equals the eager forward bit
for bit, and so do those eager forwards."""
from importlib import import_module, reload

import pytest
import torch

import dit_stack as ds
from fake_comfy import FakeLoRA, install_fake_comfy

pytestmark = pytest.mark.gpu


def same_bits(a, b):
    return a.shape == b.shape and torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


def test_forward_replays_from_a_captured_graph(gpu):
    install_fake_comfy()
    m = import_module("comfyui-int4-convrot-rdna4_amd.int4_ops")
    if m.Int4ConvRotOps is None:
        m = reload(m)
    print("graph capture: 2-block stack, 128 + 64 tokens", flush=True)
    model, _, patches, applied = ds.build_int4_stack(m.Int4ConvRotOps, FakeLoRA, depth=2)
    assert applied == set(patches)
    x = ds.synthetic_inputs(128, 64, device="cuda")
    y = ds.synthetic_inputs(600, 40, seed=5, device="cuda")          # other token counts between replays
    with torch.no_grad():
        ref = model(*x).clone()
        ref_y = model(*y).clone()
        static = [t.clone() for t in x]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            model(*static)                                            # warm-up on a side stream, as torch's capture recipe has it
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = model(*static)
        for rep in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert same_bits(out, ref), rep
            o = model(*y)
            torch.cuda.synchronize()
            assert same_bits(o, ref_y), rep
        # new values in the captured input buffers: the replay follows them
        z = ds.synthetic_inputs(128, 64, seed=9, device="cuda")
        ref_z = model(*z).clone()
        for t, v in zip(static, z):
            t.copy_(v)
        g.replay()
        torch.cuda.synchronize()
        assert same_bits(out, ref_z)
        assert not same_bits(ref_z, ref)
