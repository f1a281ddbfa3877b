"""Loader-step format adapter: alias mapping, layout and group-size detection, zero-point
mapping (CPU), and on the GPU the adapted weight's matmul against the oracle."""
import numpy as np
import pytest
import torch

from oracle import awq_oracle as O
from oracle.gen import make_awq_problem
from kernel_paths import decode_serves

DEV = torch.device("cuda:0")


def test_aliases_and_layout_detection():
    from litevllm_amd import loader
    p = make_awq_problem(M=1, K=512, N=64, group_size=64, seed=5)
    qr, zr, sr = O.repack_awq_to_ref(p["qweight"], p["qzeros"], p["scales"])
    sd = {"m.weight_packed": torch.from_numpy(qr), "m.weight_scale": torch.from_numpy(sr),
          "m.weight_zero_point": torch.from_numpy(zr), "other.qweight": torch.zeros(1)}
    c = loader.awq_components(sd, "m")
    assert set(c) == {"qweight", "scales", "qzeros"} and c["qweight"] is sd["m.weight_packed"]
    assert loader.detect_layout(c["qweight"], c["scales"]) == ("ref", 512, 64, 64)
    assert loader.detect_layout(torch.from_numpy(p["qweight"]), torch.from_numpy(p["scales"])) == ("autoawq", 512, 64, 64)
    with pytest.raises(ValueError):
        loader.detect_layout(torch.zeros(10, 3, dtype=torch.int32), torch.zeros(7, 5))


def test_unpacked_zero_points_are_packed_along_groups():
    from litevllm_amd import loader
    rng = np.random.default_rng(1)
    z = rng.integers(0, 16, size=(24, 20))
    packed = loader._pack_groups(torch.from_numpy(z))
    assert packed.shape == (24, 3) and packed.dtype == torch.int32
    assert np.array_equal(O.unpack_ref(packed.numpy())[:, :20], z)
    zz = loader._zeros_for(torch.from_numpy(z), "ref", K=20 * 32, N=24, G=32)
    assert torch.equal(zz, packed)


def test_symmetric_module_gives_packed_int4_weight():
    from litevllm_amd import loader
    from litevllm_amd.tensor import PackedInt4Weight
    qw = torch.zeros(16, 8, dtype=torch.int32)
    sc = torch.ones(16, 2, dtype=torch.float16)
    w = loader.make_awq_weight({"qweight": qw, "scales": sc, "weight_shape": torch.tensor([16, 64])}, to_autoawq=False)
    assert isinstance(w, PackedInt4Weight) and w.layout == "ref" and w.group_size == 32
    assert w.original_shape == (16, 64)


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["compressed_packed_zp", "compressed_unpacked_zp", "unpacked_zp_u8", "autoawq",
                                 "symmetric"])
@pytest.mark.parametrize("M", [1, 40])
def test_adapted_weight_matmul(fmt, M):
    from litevllm_amd import loader
    print(f"loader fmt={fmt} M={M}", flush=True)
    K, N, G = 1024, 256, 128
    p = make_awq_problem(M=M, K=K, N=N, group_size=G, seed=7)
    qr, zr, sr = O.repack_awq_to_ref(p["qweight"], p["qzeros"], p["scales"])
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    if fmt == "autoawq":
        comps = {"qweight": t(p["qweight"]), "scales": t(p["scales"]), "qzeros": t(p["qzeros"])}
    elif fmt == "compressed_packed_zp":
        comps = {"qweight": t(qr), "scales": t(sr), "qzeros": t(zr)}
    elif fmt == "compressed_unpacked_zp":
        # compressed-tensors' signed int4 convention: int8 zero points in [-8, 7], weights stored +8
        zs = O.unpack_ref(zr)[:, : K // G].astype(np.int64) - 8
        comps = {"qweight": t(qr), "scales": t(sr), "qzeros": t(zs.astype(np.int8))}
    elif fmt == "unpacked_zp_u8":
        comps = {"qweight": t(qr), "scales": t(sr), "qzeros": t(O.unpack_ref(zr)[:, : K // G].astype(np.uint8))}
    else:
        comps = {"qweight": t(qr), "scales": t(sr)}
    w = loader.make_awq_weight(comps, device=DEV, prepare_decode=True)
    assert w.layout == "autoawq"
    # no prefix and no profile hint: the reference's default scope (attention_only) would take the
    # dense path, so ask for the fused one
    y = w.matmul(t(p["x"]).to(DEV), config={"kernel_policy": {"awq_fused_scope": "all"}}).float().cpu().numpy()
    zp = fmt != "symmetric"
    wd = O.dequant_awq(p["qweight"], p["scales"], p["qzeros"] if zp else None, G,
                       out_dtype="float32" if decode_serves(M, N, G) else "float16", zero_point=zp)
    rep = O.error_report(y, O.linear_exact(p["x"], wd.T))
    assert rep["max_ulp"] <= 1.0, rep
