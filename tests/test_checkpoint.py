"""CPU checks of the FP8 checkpoint helpers: layout, validation and a
safetensors round trip (quantised with the torch reference quantiser)."""
import pytest
import torch

from hf_kernels_helion_amd.finegrained_fp8_helion import checkpoint, synthetic


def _ckpt():
    g = torch.Generator().manual_seed(1)
    W1 = torch.randn(256, 384, generator=g) * 0.02
    W2 = torch.randn(130, 260, generator=g) * 0.02
    q1, s1 = synthetic.quantize_weight_blockwise(W1)
    q2, s2 = synthetic.quantize_weight_blockwise(W2)
    return {"l1.weight": q1, "l1.weight_scale_inv": s1, "l2.weight": q2,
            "l2.weight_scale_inv": s2, "norm.weight": torch.ones(384)}


def test_roundtrip_and_pairs(tmp_path):
    sd = _ckpt()
    p = tmp_path / "model.safetensors"
    checkpoint.save_fp8_checkpoint(p, sd)
    back = checkpoint.load_fp8_checkpoint(p)
    assert set(back) == set(sd)
    for k in sd:
        assert back[k].dtype == sd[k].dtype
        assert torch.equal(back[k].view(torch.uint8) if back[k].dtype == torch.float8_e4m3fn
                           else back[k], sd[k].view(torch.uint8)
                           if sd[k].dtype == torch.float8_e4m3fn else sd[k])
    pairs = checkpoint.fp8_linear_weights(back)
    assert set(pairs) == {"l1.weight", "l2.weight"}
    assert pairs["l2.weight"][1].shape == (2, 3)


def test_validation_errors():
    sd = _ckpt()
    del sd["l1.weight_scale_inv"]
    with pytest.raises(ValueError, match="without"):
        checkpoint.fp8_linear_weights(sd)
    sd = _ckpt()
    sd["l2.weight_scale_inv"] = torch.ones(3, 3)
    with pytest.raises(ValueError, match="expected float32"):
        checkpoint.fp8_linear_weights(sd)
