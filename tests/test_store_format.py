"""CPU tests of the on-disk formats: experts.bin / experts.idx (format 2.0),
the legacy per-expert files with metadata.json (format 1.0), and the
legacy -> single-blob converter.

What pins them: the reference's format as its writers lay it out
(preprocess/pack_glm4.py:72-141, cache/packed_expert_store.py:627-739,
preprocess/pack_weights.py:271-449) — JSON keys, a 20-byte header of five
u32, six tensors back to back — and the blob sizes the reference's shape
tables give at Mixtral and GLM-4.5-Air dims.
"""
import json
import os
import struct

import numpy as np
import pytest
import torch

import oracle
from hydranet_amd.cache.blob_layout import BlobLayout
from hydranet_amd.cache.packed_expert_store import GpuExpertSlot, PackedExpertStore
from hydranet_amd.preprocess import pack_store as ps
from tests._store import make_store, random_expert


def test_blob_sizes_at_model_dims():
    # Mixtral: 3 x 14336 x 2048 packed + 3 x 917504 B of scales; 256 blobs = 23.25 GB
    mix = BlobLayout.from_dims(4096, 14336, 128)
    assert mix.total_size == 3 * 14336 * 2048 + 3 * 917504 == 90832896
    assert round(256 * mix.total_size / 1e9, 2) == 23.25
    # GLM-4.5-Air routed experts: down scales are [4096, 11] fp16 (22-byte rows)
    glm = BlobLayout.from_dims(4096, 1408, 128)
    assert glm.down_scales_size == 4096 * 11 * 2
    assert glm.total_size == 8921088
    assert 45 * 128 * glm.total_size == 51_385_466_880  # 5760 blobs, 51.38 GB


def test_index_schema_and_blob_bytes(tmp_path):
    experts = make_store(tmp_path, num_layers=2, num_experts=3, model_type="glm4_air")
    idx = json.loads((tmp_path / "experts.idx").read_text())
    assert idx["format_version"] == "2.0" and idx["model_type"] == "glm4_air"
    assert idx["quant_config"] == {"bits": 4, "group_size": 128, "symmetric": True}
    assert idx["model_config"] == {"num_layers": 2, "num_experts": 3, "hidden_dim": 256,
                                   "intermediate_dim": 512}
    size = BlobLayout.from_dims(256, 512, 128).total_size
    assert [(e["layer_idx"], e["expert_idx"]) for e in idx["experts"]] == \
        [(l, e) for l in range(2) for e in range(3)]
    assert [e["offset"] for e in idx["experts"]] == [i * size for i in range(6)]
    assert all(e["size"] == size for e in idx["experts"])
    raw = (tmp_path / "experts.bin").read_bytes()
    assert len(raw) == 6 * size
    # each blob is the six tensors' bytes back to back in blob order
    for i, (key, t) in enumerate(experts.items()):
        want = b"".join(t[n].numpy().tobytes() for n in ("gate_packed", "gate_scales",
                                                           "up_packed", "up_scales",
                                                           "down_packed", "down_scales"))
        assert raw[i * size:(i + 1) * size] == want, key


def test_no_model_type_key_when_absent(tmp_path):
    make_store(tmp_path, num_layers=1, num_experts=1)
    assert "model_type" not in json.loads((tmp_path / "experts.idx").read_text())


@pytest.mark.parametrize("use_mmap", [True, False])
def test_reader_round_trip(tmp_path, use_mmap):
    experts = make_store(tmp_path, num_layers=2, num_experts=2)
    store = PackedExpertStore(tmp_path / "experts.idx", device=torch.device("cpu"),
                              use_mmap=use_mmap)
    assert store.hidden_dim == 256 and store.intermediate_dim == 512 and store.group_size == 128
    for (l, e), t in experts.items():
        slot = GpuExpertSlot(0, 256, 512, 128, torch.device("cpu"))
        store.load_to_gpu_slot(l, e, slot)
        for n, v in t.items():
            assert torch.equal(getattr(slot, n), v), (l, e, n)
    got = {(l, e): t for l, e, t in ps.iter_store_experts(store)}
    assert set(got) == set(experts)
    assert all(torch.equal(got[k][n], experts[k][n]) for k in experts for n in experts[k])
    with pytest.raises(ValueError, match="not in index"):
        store.get_expert_blob(5, 0)
    store.close()


def test_writer_checks_shapes_and_duplicates(tmp_path):
    t = random_expert(1, 256, 512, 128)
    with ps.ExpertStoreWriter(tmp_path, 1, 2, 256, 512, 128) as w:
        w.add(0, 0, t)
        with pytest.raises(ValueError, match="twice"):
            w.add(0, 0, t)
        bad = dict(t, down_scales=t["down_scales"][:, :2].contiguous())
        with pytest.raises(ValueError, match="down_scales"):
            w.add(0, 1, bad)
        with pytest.raises(ValueError, match="blob of"):
            w.add(0, 1, b"\0" * 10)


def test_quantized_expert_round_trip(tmp_path):
    """Experts quantised with the packer rule survive write -> read bit for bit
    and dequantise to the same fp16 values."""
    H, I, g = 256, 384, 128
    rng = np.random.default_rng(3)
    t = {}
    for pre, (n, k) in (("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float16)
        p, s = oracle.quantize(w, g, mode=0)
        t[f"{pre}_packed"], t[f"{pre}_scales"] = torch.from_numpy(p), torch.from_numpy(s.copy())
    ps.write_packed_store(tmp_path, [(0, 0, t)], 1, 1, H, I, g)
    store = PackedExpertStore(tmp_path / "experts.idx", device=torch.device("cpu"))
    blob, _ = store.get_expert_blob(0, 0)
    back = ps.blob_tensors(blob, H, I, g)
    for pre in ("gate", "up", "down"):
        a = oracle.dequant(back[f"{pre}_packed"].numpy(), back[f"{pre}_scales"].numpy(), g)
        b = oracle.dequant(t[f"{pre}_packed"].numpy(), t[f"{pre}_scales"].numpy(), g)
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    store.close()


def _legacy_experts(L, E, H, I, g):
    return [ps.PackedExpert.from_blob_tensors(l, e, random_expert(77 + 10 * l + e, H, I, g), g,
                                              checksum=f"{l}{e}")
            for l in range(L) for e in range(E)]


def test_legacy_file_layout(tmp_path):
    p = _legacy_experts(1, 1, 256, 512, 128)[0]
    n = ps.save_packed_expert(p, tmp_path / "x.bin")
    raw = (tmp_path / "x.bin").read_bytes()
    size = BlobLayout.from_dims(256, 512, 128).total_size
    assert n == size == p.size_bytes() and len(raw) == 20 + size
    assert struct.unpack("<IIIII", raw[:20]) == (0, 0, 256, 512, 128)
    assert raw[20:] == ps.expert_blob(p).tobytes()
    q = ps.load_packed_expert(tmp_path / "x.bin")
    assert (q.layer_idx, q.expert_idx, q.hidden_dim, q.intermediate_dim, q.group_size) == \
        (0, 0, 256, 512, 128)
    for a, b in zip(p.blob_tensors().values(), q.blob_tensors().values()):
        assert torch.equal(a, b)
    assert q.gate_proj_scales.dtype == torch.float16 and q.down_proj_packed.shape == (256, 256)


def test_legacy_metadata_and_conversion(tmp_path):
    L, E, H, I, g = 2, 3, 256, 512, 128
    experts = _legacy_experts(L, E, H, I, g)
    meta = ps.write_legacy_store(experts, tmp_path / "legacy", L, E)
    assert meta["format_version"] == "1.0"
    m = json.loads((tmp_path / "legacy" / "metadata.json").read_text())
    assert m["experts"][4] == {"layer": 1, "expert": 1, "file": "expert_L01_E01.bin",
                               "size_bytes": BlobLayout.from_dims(H, I, g).total_size,
                               "checksum": "11"}
    assert m["total_size_bytes"] == L * E * BlobLayout.from_dims(H, I, g).total_size
    assert m["model_config"] == {"num_layers": L, "num_experts": E, "hidden_dim": H,
                                 "intermediate_dim": I}
    idx = ps.pack_to_single_blob(tmp_path / "legacy", tmp_path / "v2", L, E, H, I, g)
    assert idx["format_version"] == "2.0" and len(idx["experts"]) == L * E
    raw = (tmp_path / "v2" / "experts.bin").read_bytes()
    # conversion is a byte copy of each legacy payload, in (layer, expert) order
    want = b"".join((tmp_path / "legacy" / ps.legacy_expert_filename(l, e)).read_bytes()[20:]
                    for l in range(L) for e in range(E))
    assert raw == want


def test_legacy_errors(tmp_path):
    L, E, H, I, g = 1, 2, 256, 512, 128
    ps.write_legacy_store(_legacy_experts(L, E, H, I, g), tmp_path / "a", L, E)
    (tmp_path / "a" / "expert_L00_E01.bin").unlink()
    with pytest.raises(FileNotFoundError, match="expert_L00_E01"):
        ps.pack_to_single_blob(tmp_path / "a", tmp_path / "b", L, E, H, I, g)
    path = tmp_path / "a" / "expert_L00_E00.bin"
    raw = path.read_bytes()
    path.write_bytes(raw[:-1])
    with pytest.raises(ValueError, match="payload bytes"):
        ps.load_packed_expert(path)
    path.write_bytes(raw)
    with pytest.raises(ValueError, match="does not match"):
        ps.pack_to_single_blob(tmp_path / "a", tmp_path / "c", 1, 1, H, 256, g)


def test_checksum_known_answer():
    w = {"gate_proj": torch.ones(4, 8, dtype=torch.float16),
         "up_proj": torch.full((4, 8), -2.0, dtype=torch.float16),
         "down_proj": torch.full((8, 4), 0.5, dtype=torch.float16)}
    # 32 + 64 + 16 = 112.0 -> float64 bits 0x405c000000000000, little-endian hex
    assert ps.compute_expert_checksum(w) == "0000000000005c40"
    assert ps.verify_expert_checksum(w, "0000000000005c40")
    assert not ps.verify_expert_checksum(dict(w, down_proj=w["down_proj"].t()), "00")


# ---------------------------------------------------------------- files the reference wrote
_REF_STORE = os.path.join(os.path.dirname(__file__), "golden", "store_format")


def _ref_case():
    with open(os.path.join(_REF_STORE, "legacy_files.json")) as f:
        return json.load(f)


def _seeded_packed_experts():
    """PackedExperts of the fixture's seeded weights, packed by the oracle packer
    (pinned against the reference packer by tests/test_oracle.py)."""
    import sys
    gold = os.path.join(os.path.dirname(__file__), "golden")
    if gold not in sys.path:
        sys.path.insert(0, gold)
    import gen
    import oracle
    from hydranet_amd.preprocess.pack_store import PackedExpert, compute_expert_checksum
    c = _ref_case()["case"]
    out = []
    for layer in range(c["L"]):
        for e in range(c["E"]):
            w = gen.expert_weights(c["seed"], e, c["H"], c["I"], layer=layer)
            t = {}
            for proj, pre in (("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
                p, s = oracle.quantize(w[proj], c["g"], mode=0)
                t[f"{pre}_packed"] = torch.from_numpy(np.ascontiguousarray(p))
                t[f"{pre}_scales"] = torch.from_numpy(np.ascontiguousarray(s))
            ck = compute_expert_checksum({k: torch.from_numpy(v) for k, v in w.items()})
            out.append(PackedExpert.from_blob_tensors(layer, e, t, c["g"], ck))
    return c, out


def test_reader_reads_reference_single_blob_bit_for_bit():
    """experts.bin / experts.idx written by the reference's pack_to_single_blob
    (cache/packed_expert_store.py:627-739) read back through PackedExpertStore."""
    from hydranet_amd.cache.packed_expert_store import PackedExpertStore
    from hydranet_amd.preprocess.pack_store import iter_store_experts
    c, experts = _seeded_packed_experts()
    st = PackedExpertStore(os.path.join(_REF_STORE, "experts.idx"), device=torch.device("cpu"))
    try:
        assert st.format_version == "2.0"
        assert (st.hidden_dim, st.intermediate_dim, st.group_size) == (c["H"], c["I"], c["g"])
        got = {(l, e): t for l, e, t in iter_store_experts(st)}
        assert len(got) == len(experts)
        for pe in experts:
            t = got[(pe.layer_idx, pe.expert_idx)]
            for name, ref in pe.blob_tensors().items():
                assert torch.equal(t[name].view(torch.uint8).reshape(-1),
                                   ref.contiguous().view(torch.uint8).reshape(-1)), name
    finally:
        st.close()


def test_writers_reproduce_reference_files_byte_for_byte(tmp_path):
    """Legacy files (pack_mixtral_experts, preprocess/pack_weights.py:271-381),
    their metadata.json and the converted experts.bin/.idx equal the reference's."""
    from hydranet_amd.preprocess.pack_store import (load_packed_expert, pack_to_single_blob,
                                                    write_legacy_store)
    c, experts = _seeded_packed_experts()
    legacy = tmp_path / "legacy"
    meta = write_legacy_store(experts, legacy, c["L"], c["E"])
    with open(os.path.join(_REF_STORE, "metadata.json")) as f:
        assert meta == json.load(f)   # checksums included (pack_weights.py:36-50)
    import hashlib
    for name, digest in _ref_case()["sha256"].items():
        assert hashlib.sha256((legacy / name).read_bytes()).hexdigest() == digest, name
        # and the legacy reader parses what the reference wrote
        pe = load_packed_expert(legacy / name)
        assert (pe.hidden_dim, pe.intermediate_dim, pe.group_size) == (c["H"], c["I"], c["g"])
    idx = pack_to_single_blob(legacy, tmp_path / "blob", c["L"], c["E"], c["H"], c["I"], c["g"])
    ref_bin = open(os.path.join(_REF_STORE, "experts.bin"), "rb").read()
    assert (tmp_path / "blob" / "experts.bin").read_bytes() == ref_bin
    with open(os.path.join(_REF_STORE, "experts.idx")) as f:
        assert idx == json.load(f)
