"""Checkpoint ingest: name rules, the safetensors reader, and (GPU) loading a
layer's tables with the finite-bit gate."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from glm_moe.model_loader import placement as P
from glm_moe.model_loader.safetensors_io import SafetensorsFile, write_safetensors


# ----------------------------------------------------------------------------- names (CPU)
def test_routed_source_names_follow_the_reference():
    # tests/model_loader/test_placement.py:36-57 of the reference: expert 130 of layer 3
    src = P.routed_source("model.layers.3.mlp.experts.130.gate_proj.weight")
    assert src == (3, 130, "gate_proj", "weight")
    assert P.runtime_name("model.layers.3.mlp.experts.130.gate_proj.weight", "F8_E4M3") == \
        "model.layers.3.mlp.experts.gate_proj.weight_bits"
    assert P.runtime_name("model.layers.3.mlp.experts.130.gate_proj.weight_scale_inv", "F32") == \
        "model.layers.3.mlp.experts.gate_proj.scale_inv"
    # expert axis of eight: coordinate 130 // 32 = 4 (slots 16..19), local index 130 % 32 = 2
    assert P.expert_coordinate(130, 256, 8) == (4, 2)
    assert P.expert_coordinate(130, 256, 1) == (0, 130)
    assert P.runtime_name("model.layers.3.mlp.shared_experts.down_proj.weight", "F8_E4M3") == \
        "model.layers.3.mlp.shared_experts.down_proj.weight_bits"
    assert P.runtime_name("model.layers.0.mlp.down_proj.weight", "F8_E4M3") == "model.layers.0.mlp.down_proj.weight_bits"
    assert P.runtime_name("model.layers.3.mlp.gate.weight", "BF16") == "model.layers.3.mlp.gate.weight"
    assert P.runtime_name("model.layers.3.mlp.gate.e_score_correction_bias", "F32") == \
        "model.layers.3.mlp.gate.e_score_correction_bias"
    # a BF16 .weight keeps its name: only FP8 payloads become weight_bits
    assert P.runtime_name("model.layers.3.mlp.shared_experts.down_proj.weight", "BF16").endswith(".weight")
    assert P.routed_source("model.layers.3.mlp.experts.gate_proj.weight") is None
    assert P.routed_source("model.layers.3.mlp.experts.7.gate_proj.bias") is None
    with pytest.raises(ValueError, match="divide"):
        P.expert_coordinate(0, 255, 8)
    with pytest.raises(ValueError, match="outside"):
        P.expert_coordinate(256, 256, 8)


# ----------------------------------------------------------------------------- safetensors (CPU)
def test_reader_and_writer_agree_with_the_safetensors_library(tmp_path):
    from safetensors.numpy import load_file, save_file

    rng = np.random.default_rng(0)
    arrays = {"a.f32": rng.standard_normal((3, 5)).astype(np.float32),
              "b.u8": rng.integers(0, 255, (7, 9), dtype=np.uint8),
              "c.i32": rng.integers(-9, 9, (4,), dtype=np.int32)}
    theirs = tmp_path / "theirs.safetensors"
    save_file(arrays, str(theirs))
    f = SafetensorsFile(theirs)
    assert {n: f.info(n).dtype for n in arrays} == {"a.f32": "F32", "b.u8": "U8", "c.i32": "I32"}
    for n, a in arrays.items():
        np.testing.assert_array_equal(f.array(n), a)
    ours = tmp_path / "ours.safetensors"
    write_safetensors(ours, {"a.f32": ("F32", arrays["a.f32"]), "b.u8": ("U8", arrays["b.u8"]),
                             "c.i32": ("I32", arrays["c.i32"])}, metadata={"format": "pt"})
    back = load_file(str(ours))
    for n, a in arrays.items():
        np.testing.assert_array_equal(back[n], a)
    # FP8 and BF16 payloads are raw bytes with their own dtype tags
    bits = rng.integers(0, 126, (4, 8), dtype=np.uint8)
    bf16 = rng.integers(0, 1 << 15, (2, 3), dtype=np.uint16)
    write_safetensors(ours, {"w": ("F8_E4M3", bits), "h": ("BF16", bf16)})
    g = SafetensorsFile(ours)
    assert g.info("w").dtype == "F8_E4M3" and g.info("h").dtype == "BF16"
    np.testing.assert_array_equal(g.array("w"), bits)
    np.testing.assert_array_equal(g.array("h"), bf16)


def test_reader_refuses_inconsistent_files(tmp_path):
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(b"\x05\x00")
    with pytest.raises(ValueError, match="short header"):
        SafetensorsFile(bad)
    import json
    import struct

    header = json.dumps({"x": {"dtype": "F32", "shape": [4], "data_offsets": [0, 8]}}).encode()
    bad.write_bytes(struct.pack("<Q", len(header)) + header + b"\x00" * 8)
    with pytest.raises(ValueError, match="inconsistent offsets"):
        SafetensorsFile(bad)
    header = json.dumps({"x": {"dtype": "C64", "shape": [1], "data_offsets": [0, 8]}}).encode()
    bad.write_bytes(struct.pack("<Q", len(header)) + header + b"\x00" * 8)
    with pytest.raises(ValueError, match="unsupported dtype"):
        SafetensorsFile(bad)


def test_loader_refuses_a_cpu_device(tmp_path):
    from glm_moe.model_loader import load_moe_layer

    with pytest.raises(ValueError, match="GPU"):
        load_moe_layer([], 0, device="cpu", num_experts=8, hidden_size=256, intermediate_size=256)


# ----------------------------------------------------------------------------- GPU ingest
def _write_layer(path, layer, tables, shared, router_w, bias, plant=None):
    """Per-expert source tensors with the checkpoint's names, over two files."""
    experts = tables["gate_bits"].shape[0]
    names = {"gate": "gate_proj", "up": "up_proj", "down": "down_proj"}
    files = [{}, {}]
    for e in range(experts):
        for short, proj in names.items():
            w, s = P.source_names(layer, e, proj)
            files[e % 2][w] = ("F8_E4M3", tables[f"{short}_bits"][e])
            files[e % 2][s] = ("F32", tables[f"{short}_scale"][e])
    for short, proj in names.items():
        w, s = P.shared_source_names(layer, proj)
        files[0][w] = ("F8_E4M3", shared[f"{short}_bits"])
        files[0][s] = ("F32", shared[f"{short}_scale"])
    w, b = P.router_source_names(layer)
    files[1][w] = ("BF16", router_w)
    files[1][b] = ("F32", bias)
    if plant is not None:
        name, index, value = plant
        for f in files:
            if name in f:
                dtype, a = f[name]
                a = a.copy()
                a.reshape(-1)[index] = value
                f[name] = (dtype, a)
    paths = []
    for i, f in enumerate(files):
        p = path / f"model-0000{i + 1}-of-00002.safetensors"
        write_safetensors(p, f)
        paths.append(p)
    return paths


@pytest.fixture(scope="module")
def tiny_layer():
    from glm_moe import synthetic as S

    cfg = S.MoeConfig("ingest", 64, 8, 256, 256, 2, 0.0)
    tables = S.host_expert_tables(cfg, 5)
    one = S.MoeConfig("shared", 1, 1, 256, 256, 1, 0.0)
    st = S.host_expert_tables(one, 6)
    shared = {k: v[0] for k, v in st.items()}
    rng = np.random.default_rng(3)
    router_w = rng.integers(0x3C00, 0x3E00, (8, 256), dtype=np.uint16)  # finite bf16 bit patterns
    bias = rng.standard_normal(8).astype(np.float32)
    return cfg, tables, shared, router_w, bias


@pytest.mark.gpu
def test_count_nonfinite_fp8_is_exact():
    from glm_moe import _lib

    rng = np.random.default_rng(11)
    for n in (1, 3, 4, 4099, 1 << 20):
        raw = rng.integers(0, 256, n, dtype=np.uint8)
        want = int(np.sum((raw & 0x7F) == 0x7F))
        bits = torch.from_numpy(raw).cuda()
        count = torch.zeros(1, dtype=torch.int64, device="cuda")
        _lib.call("glm_moe_count_nonfinite_fp8", _lib.ptr(bits), n, _lib.ptr(count), _lib.stream_of(bits))
        assert int(count.item()) == want, n


@pytest.mark.gpu
def test_loaded_layer_equals_its_source_and_runs(tmp_path, tiny_layer):
    from glm_moe import synthetic as S
    from glm_moe.layers.fp8 import dequantize_fp8_bits_block_weight
    from glm_moe.layers.moe.routed_experts import routed_experts
    from glm_moe.model_loader import load_moe_layer

    cfg, tables, shared, router_w, bias = tiny_layer
    paths = _write_layer(tmp_path, 3, tables, shared, router_w, bias)
    got = load_moe_layer(paths, 3, device="cuda", num_experts=8, hidden_size=256, intermediate_size=256)
    for k, v in zip(("gate_bits", "gate_scale", "up_bits", "up_scale", "down_bits", "down_scale"),
                    got.expert_tables()):
        np.testing.assert_array_equal(v.cpu().numpy(), tables[k])
    for short, t in (("gate", got.shared_gate), ("up", got.shared_up), ("down", got.shared_down)):
        want = dequantize_fp8_bits_block_weight(torch.from_numpy(shared[f"{short}_bits"]).cuda(),
                                                torch.from_numpy(shared[f"{short}_scale"]).cuda())
        assert torch.equal(t, want)
    np.testing.assert_array_equal(got.router_weight.view(torch.int16).cpu().numpy().view(np.uint16), router_w)
    np.testing.assert_array_equal(got.correction_bias.cpu().numpy(), bias)
    x = torch.from_numpy(S.hidden_states(cfg, 1)).to(torch.bfloat16).cuda()
    ids, w = (torch.from_numpy(a).cuda() for a in S.routes(cfg, 1))
    direct = [torch.from_numpy(tables[k]).cuda() for k in
              ("gate_bits", "gate_scale", "up_bits", "up_scale", "down_bits", "down_scale")]
    a, ok_a = routed_experts(x, ids, w, *got.expert_tables())
    b, ok_b = routed_experts(x, ids, w, *direct)
    assert bool(ok_a) and bool(ok_b) and torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.parametrize("plant,match", [
    (("model.layers.3.mlp.experts.5.down_proj.weight", 1234, 0x7F), "non-finite bits"),
    (("model.layers.3.mlp.experts.0.gate_proj.weight", 0, 0xFF), "non-finite bits"),
    (("model.layers.3.mlp.shared_experts.up_proj.weight", 77, 0xFF), "non-finite bits"),
    (("model.layers.3.mlp.experts.2.up_proj.weight_scale_inv", 1, np.float32(np.inf)), "non-finite"),
    (("model.layers.3.mlp.gate.e_score_correction_bias", 4, np.float32(np.nan)), "non-finite"),
])
def test_loader_refuses_non_finite_payloads(tmp_path, tiny_layer, plant, match):
    from glm_moe.model_loader import CheckpointValidationError, load_moe_layer

    cfg, tables, shared, router_w, bias = tiny_layer
    paths = _write_layer(tmp_path, 3, tables, shared, router_w, bias, plant=plant)
    with pytest.raises(CheckpointValidationError, match=match):
        load_moe_layer(paths, 3, device="cuda", num_experts=8, hidden_size=256, intermediate_size=256)


@pytest.mark.gpu
def test_loader_refuses_missing_and_misshapen_tensors(tmp_path, tiny_layer):
    from glm_moe.model_loader import CheckpointValidationError, load_moe_layer

    cfg, tables, shared, router_w, bias = tiny_layer
    paths = _write_layer(tmp_path, 3, tables, shared, router_w, bias)
    with pytest.raises(CheckpointValidationError, match="lacks"):
        load_moe_layer(paths[:1], 3, device="cuda", num_experts=8, hidden_size=256, intermediate_size=256)
    with pytest.raises(CheckpointValidationError, match="shape"):
        load_moe_layer(paths, 3, device="cuda", num_experts=8, hidden_size=256, intermediate_size=128)
    with pytest.raises(CheckpointValidationError, match="beyond"):
        load_moe_layer(paths, 3, device="cuda", num_experts=4, hidden_size=256, intermediate_size=256)


@pytest.mark.gpu
def test_expert_parallel_shares_sum_to_the_full_layer(tmp_path, tiny_layer):
    from glm_moe import synthetic as S
    from glm_moe.layers.moe.routed_experts import routed_experts
    from glm_moe.model_loader import load_moe_layer

    cfg, tables, shared, router_w, bias = tiny_layer
    paths = _write_layer(tmp_path, 3, tables, shared, router_w, bias)
    x = torch.from_numpy(S.hidden_states(cfg, 2)).to(torch.bfloat16).cuda()
    ids, w = (torch.from_numpy(a).cuda() for a in S.routes(cfg, 2))
    full = load_moe_layer(paths, 3, device="cuda", num_experts=8, hidden_size=256, intermediate_size=256,
                          shared=False, router=False)
    ref, ok = routed_experts(x, ids, w, *full.expert_tables())
    assert bool(ok)
    total = torch.zeros_like(ref, dtype=torch.float32)
    for rank in range(2):
        part = load_moe_layer(paths, 3, device="cuda", num_experts=8, hidden_size=256, intermediate_size=256,
                              ep_rank=rank, ep_size=2, shared=False, router=False)
        assert part.first_expert == 4 * rank and part.num_local == 4
        np.testing.assert_array_equal(part.gate_bits.cpu().numpy(), tables["gate_bits"][4 * rank:4 * rank + 4])
        y, _ = routed_experts(x, part.local_route_indices(ids), w, *part.expert_tables(), drop_unowned=True)
        total += y.float()
    # each share rounds its own partial sum to bf16 once: the shares' sum agrees to bf16 precision
    err = (total - ref.float()).abs()
    assert float(err.max()) <= 2e-2 and float(err.mean() / ref.float().abs().mean()) <= 5e-3
