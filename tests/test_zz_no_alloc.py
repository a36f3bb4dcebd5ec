"""rlq_moe_no_alloc: the MoE layer with its scratch in the library's static device array.

Called through the C ABI and checked bit for bit against rlq_moe with a caller workspace (the
existing entry point), on two calls in a row, the second with fewer tokens (the array keeps
the first call's contents), and in both orders of kernel paths (the staged expert kernel at
40 tokens, the one-token and fused down+combine launches at 1 and 3).
"""

import numpy as np
import pytest

from raceline_amd import lib
from tests.qdata import to_dev, upload_mlx

import oracle as O

pytestmark = pytest.mark.gpu


def _moe_stack(seed, E, H, I, dev):
    from raceline_amd import ops

    rng = np.random.default_rng(seed)
    Wg = rng.standard_normal(((E + 1) * 2 * I, H), dtype=np.float32) * np.float32(0.02)
    Wd = rng.standard_normal(((E + 1) * H, I), dtype=np.float32) * np.float32(0.02)
    gu, dn = O.quantize_affine_rtn(Wg, "f16"), O.quantize_affine_rtn(Wd, "f16")
    return ops.pack_moe(upload_mlx(*gu, "f16", dev), upload_mlx(*dn, "f16", dev), E, H, I)


def _layer(entry, x, logits, mw, topk, h, ws=None):
    import torch

    stream = torch.cuda.current_stream().cuda_stream
    args = [x.data_ptr(), x.stride(0), logits.data_ptr(), logits.stride(0), x.shape[0], mw.E, topk, 1, mw.H, mw.I,
            mw.gate_up.packed.data_ptr(), mw.down.packed.data_ptr(), mw.gate_up.code, h.data_ptr(), h.stride(0)]
    if entry == "rlq_moe":
        args += [ws.data_ptr(), ws.numel()]
    lib.call(entry, *args, stream)


@pytest.mark.parametrize("order", [(40, 3), (3, 1), (40, 1)])
def test_no_alloc_matches_workspace_entry(gpu, order):
    import torch

    E, H, I, topk = 64, 1024, 256, 8
    mw = _moe_stack(7, E, H, I, gpu)
    rng = np.random.default_rng(8)
    for T in order:
        x = to_dev(rng.standard_normal((T, H)).astype(np.float16), gpu)
        logits = to_dev(rng.standard_normal((T, E + 1)).astype(np.float32), gpu)
        h0 = rng.standard_normal((T, H)).astype(np.float32)
        h_ref, h_new = to_dev(h0, gpu), to_dev(h0, gpu)
        ws = torch.empty(int(lib.load().rlq_moe_workspace_bytes(T, E, topk, H, I)), dtype=torch.uint8, device=gpu)
        _layer("rlq_moe", x, logits, mw, topk, h_ref, ws)
        _layer("rlq_moe_no_alloc", x, logits, mw, topk, h_new)
        torch.cuda.synchronize()
        assert torch.equal(h_new, h_ref), f"T={T}: rlq_moe_no_alloc differs from rlq_moe"


def test_no_alloc_full_size_then_decode(gpu):
    """The BASELINE MoE shapes (H=2048, I=512, E=256, top-8): 512 tokens, then one."""
    import torch

    from raceline_amd import ops, synth

    E, H, I, topk = 256, 2048, 512, 8
    assert lib.load().rlq_moe_workspace_bytes(512, E, topk, H, I) <= lib.load().rlq_moe_no_alloc_max_bytes()
    mw = ops.pack_moe(synth.random_affine((E + 1) * 2 * I, H, 11, gpu, packed=False),
                      synth.random_affine((E + 1) * H, I, 12, gpu, packed=False), E, H, I)
    for T, seed in ((512, 13), (1, 14)):
        x = synth.random_activations(T, H, seed, gpu)
        g = torch.Generator(device=gpu)
        g.manual_seed(seed)
        logits = torch.randn((T, E + 1), generator=g, device=gpu, dtype=torch.float32)
        h_ref = torch.zeros((T, H), dtype=torch.float32, device=gpu)
        h_new = torch.zeros((T, H), dtype=torch.float32, device=gpu)
        ws = torch.empty(int(lib.load().rlq_moe_workspace_bytes(T, E, topk, H, I)), dtype=torch.uint8, device=gpu)
        _layer("rlq_moe", x, logits, mw, topk, h_ref, ws)
        _layer("rlq_moe_no_alloc", x, logits, mw, topk, h_new)
        torch.cuda.synchronize()
        assert torch.equal(h_new, h_ref), f"T={T}: rlq_moe_no_alloc differs from rlq_moe"
