"""Real-trace input format (reference benchmark_mps.py:26-47): a torch.save
dict of means2d/conics/colors/opacities/depths, [G,...] or [B,G,...]."""
import pytest
import torch

from torch_gsplat_bridge_fast.scenes import load_trace


def _trace(B=None, G=50):
    g = torch.Generator().manual_seed(0)
    shape = (G,) if B is None else (B, G)
    return {
        "means2d": torch.rand(*shape, 2, generator=g, dtype=torch.float64) * 64,
        "conics": torch.rand(*shape, 3, generator=g),
        "colors": torch.rand(*shape, 3, generator=g),
        "opacities": torch.rand(*shape, generator=g),
        "depths": torch.rand(*shape, generator=g),
    }


def test_unbatched_trace_becomes_batch_one(tmp_path):
    d = _trace()
    f = tmp_path / "t.pt"
    torch.save(d, f)
    sc = load_trace(str(f))
    assert sc["means2d"].shape == (1, 50, 2) and sc["opacities"].shape == (1, 50)
    assert all(v.dtype == torch.float32 and v.is_contiguous() for v in sc.values())
    torch.testing.assert_close(sc["means2d"][0], d["means2d"].float())


def test_batched_trace_truncation(tmp_path):
    d = _trace(B=3, G=40)
    f = tmp_path / "t.pt"
    torch.save(d, f)
    sc = load_trace(str(f), batch=2, gaussians=10)
    assert sc["conics"].shape == (2, 10, 3)
    torch.testing.assert_close(sc["depths"], d["depths"][:2, :10])
    sc = load_trace(str(f), batch=9, gaussians=0)     # larger than the trace: all of it
    assert sc["colors"].shape == (3, 40, 3)


def test_missing_key_and_non_tensor_payload(tmp_path):
    d = _trace()
    del d["depths"]
    f = tmp_path / "t.pt"
    torch.save(d, f)
    with pytest.raises(ValueError, match="missing 'depths'"):
        load_trace(str(f))
    with pytest.raises(ValueError, match="required"):
        load_trace("")


def test_pickled_objects_are_refused(tmp_path):
    # a picklable object outside the weights-only allow-list
    from fractions import Fraction
    import pickle
    f = tmp_path / "t.pt"
    torch.save({"means2d": Fraction(1, 2)}, f)
    with pytest.raises(pickle.UnpicklingError):
        load_trace(str(f))
