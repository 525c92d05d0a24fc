"""Installed expert files (CPU): the loader of whallm_amd/blob_loader.py over synthetic
directories in the reference's on-disk format (manifest.py:21-42, :150-175). The pool must
hold each expert's blob in slot order byte for byte (DeepSeek rewritten to w3 | w1 | scales |
w2 | scale as the reference's fused slot, expert_layout.py:8-62), the tables must address
the right regions, and malformed directories must be refused as InstalledModel.open does."""
import json

import numpy as np
import pytest

from install_files import slot_blob, write_install
from oracle import moe as M
from whallm_amd.blob_loader import ExpertFiles
from whallm_amd.slot_cache import qwen_blob_bytes

H, I = 256, 128


@pytest.mark.parametrize("kind", ["qwen", "deepseek"])
def test_pool_holds_slot_order_blobs(tmp_path, kind):
    layers, experts = 3, 8
    src = write_install(tmp_path, kind, layers, experts, H, I, seed=1)
    files = ExpertFiles(tmp_path)
    assert (files.kind, files.layers, files.experts, files.hidden, files.inter) == (kind, layers, experts, H, I)
    assert files.blob == qwen_blob_bytes(H, I)
    assert files.in_slot_order == (kind == "qwen")
    pool = files.read(pinned=False).numpy().reshape(layers, experts, files.blob)
    for layer in range(layers):
        for e in range(experts):
            assert np.array_equal(pool[layer, e], slot_blob(kind, src[layer], e)), (layer, e)
    # a subset of layers, in the order asked for
    sub = files.read([2, 0], pinned=False).numpy().reshape(2, experts, files.blob)
    assert np.array_equal(sub[0], pool[2]) and np.array_equal(sub[1], pool[0])


def test_region_order_in_the_file_does_not_matter(tmp_path):
    a, b = tmp_path / "a", tmp_path / "b"
    write_install(a, "qwen", 1, 4, H, I, seed=2)
    write_install(b, "qwen", 1, 4, H, I, seed=2, order=[3, 1, 2, 0])
    fa, fb = ExpertFiles(a), ExpertFiles(b)
    assert fa.in_slot_order and not fb.in_slot_order
    assert np.array_equal(fa.read(pinned=False).numpy(), fb.read(pinned=False).numpy())


@pytest.mark.parametrize("kind", ["qwen", "deepseek"])
def test_tables_address_the_regions(tmp_path, kind):
    experts = 5
    src = write_install(tmp_path, kind, 2, experts, H, I, seed=3)[1]
    files = ExpertFiles(tmp_path)
    t = files.table(files.read(pinned=False), 1, swiglu_limit=7.0)
    assert t.up_first == (kind == "deepseek") and t.swiglu_limit == 7.0 and t.count == experts
    assert (t.hidden, t.inter) == (H, I)
    gu = t.gate_up.numpy().view(np.uint8).reshape(experts, -1)
    gus = t.gate_up_scales.numpy().reshape(experts, -1)
    dn = t.down.numpy().view(np.uint8).reshape(experts, -1)
    dns = t.down_scales.numpy().reshape(experts, -1)
    if kind == "qwen":
        want = (src["gate_up.weight"], src["gate_up.scale"], src["down.weight"], src["down.scale"])
    else:   # w13 = [w3 (up); w1 (gate)], rows of H/2 bytes and H/32 scales
        want = (np.concatenate([src["w3.weight"], src["w1.weight"]], 1),
                np.concatenate([src["w3.scale"], src["w1.scale"]], 1), src["w2.weight"], src["w2.scale"])
    for got, w in zip((gu, gus, dn, dns), want):
        assert np.array_equal(got, w)


def test_deepseek_table_computes_gate_from_w1(tmp_path):
    """The up_first table through the oracle equals the expert built gate-first from the
    source regions: gate = w1, up = w3, down = w2 (model.py:516-523)."""
    experts, T = 3, 4
    src = write_install(tmp_path, "deepseek", 1, experts, H, I, seed=4)[0]
    files = ExpertFiles(tmp_path)
    t = files.table(files.read(pinned=False), 0)
    x = np.random.default_rng(5).standard_normal((T, H)).astype(np.float32)
    for e in range(experts):
        loaded = M.MXFP4Expert(t.gate_up[e].numpy().view(np.uint32), t.gate_up_scales[e].numpy(),
                               t.down[e].numpy().view(np.uint32), t.down_scales[e].numpy())
        direct = M.MXFP4Expert(
            np.concatenate([src["w1.weight"][e], src["w3.weight"][e]]).view(np.uint32).reshape(2 * I, H // 8),
            np.concatenate([src["w1.scale"][e], src["w3.scale"][e]]).reshape(2 * I, H // 32),
            src["w2.weight"][e].view(np.uint32).reshape(H, I // 8), src["w2.scale"][e].reshape(H, I // 32))
        for limit in (0.0, 1.5):
            got = M.expert_ffn(x, loaded, limit=limit, up_first=True)
            want = M.expert_ffn(x, direct, limit=limit, up_first=False)
            np.testing.assert_array_equal(got, want)
        # the swap matters: reading the table gate-first gives a different expert
        assert not np.allclose(M.expert_ffn(x, loaded, up_first=False), M.expert_ffn(x, direct))


def _edit_manifest(root, fn):
    m = json.loads((root / "manifest.json").read_text())
    fn(m)
    (root / "manifest.json").write_text(json.dumps(m))


def _drop_region(m):
    m["expertRegions"].pop()


def _gap(m):
    m["expertRegions"][1]["offset"] += 4


def _dup(m):
    m["files"].append(dict(m["files"][0]))


def _size(m):
    m["files"][0]["size"] += 1


def _hole(m):
    m["files"] = [f for f in m["files"] if f["path"] != "experts/layer_00.bin"]


def _shape(m):
    m["expertRegions"][2]["shape"] = [H, I // 4]


@pytest.mark.parametrize("edit,match", [
    (_drop_region, "required regions"), (_gap, "partition"), (_dup, "duplicate"), (_size, "invalid size|does not match"),
    (_hole, "contiguous"), (_shape, "shapes"),
])
def test_malformed_installs_are_refused(tmp_path, edit, match):
    write_install(tmp_path, "qwen", 2, 4, H, I, seed=6)
    _edit_manifest(tmp_path, edit)
    with pytest.raises(ValueError, match=match):
        ExpertFiles(tmp_path)


def test_missing_short_and_escaping_files_are_refused(tmp_path):
    write_install(tmp_path, "deepseek", 2, 4, H, I, seed=7)
    layer = tmp_path / "experts" / "layer_01.bin"
    data = layer.read_bytes()
    layer.write_bytes(data[:-1])
    with pytest.raises(ValueError, match="size does not match"):
        ExpertFiles(tmp_path)
    layer.unlink()
    with pytest.raises(ValueError, match="unsafe or missing"):
        ExpertFiles(tmp_path)
    (tmp_path.parent / "elsewhere.bin").write_bytes(data)
    layer.symlink_to(tmp_path.parent / "elsewhere.bin")
    with pytest.raises(ValueError, match="unsafe or missing"):
        ExpertFiles(tmp_path)
    layer.unlink()
    layer.write_bytes(data)
    files = ExpertFiles(tmp_path)
    with pytest.raises(ValueError, match="out of range"):
        files.read([2], pinned=False)


def test_scatter_reads_resume_after_short_reads(tmp_path, monkeypatch):
    """A read that returns fewer bytes than asked continues where it stopped, mid-buffer."""
    import os
    from whallm_amd import blob_loader
    write_install(tmp_path, "deepseek", 1, 6, H, I, seed=8)
    want = ExpertFiles(tmp_path).read(pinned=False).numpy().copy()
    real = os.preadv

    def trickle(fd, bufs, offset):   # at most 4 KiB + 3 bytes per call, spread over the buffers
        left, out = 4099, []
        for b in bufs:
            if not left:
                break
            take = min(left, len(b))
            out.append(b[:take])
            left -= take
        return real(fd, out, offset)

    monkeypatch.setattr(blob_loader.os, "preadv", trickle)
    assert np.array_equal(ExpertFiles(tmp_path).read(pinned=False).numpy(), want)


# The reference's expert region tables (runtime/deepseek_v4_ssd/manifest.py:21-42): name,
# dtype, shape, offset, length, with the blob size, hidden and intermediate they imply.
REFERENCE_LAYOUTS = {
    "deepseek-v4": (13_369_344, 4096, 2048, [
        ("w1.weight", "I8", [2048, 2048], 0, 4_194_304), ("w1.scale", "F8_E8M0", [2048, 128], 4_194_304, 262_144),
        ("w2.weight", "I8", [4096, 1024], 4_456_448, 4_194_304), ("w2.scale", "F8_E8M0", [4096, 64], 8_650_752, 262_144),
        ("w3.weight", "I8", [2048, 2048], 8_912_896, 4_194_304), ("w3.scale", "F8_E8M0", [2048, 128], 13_107_200, 262_144)]),
    "deepseek-v4.1": (18_800_640, 5120, 2304, [
        ("w1.weight", "I8", [2304, 2560], 0, 5_898_240), ("w1.scale", "F8_E8M0", [2304, 160], 5_898_240, 368_640),
        ("w2.weight", "I8", [5120, 1152], 6_266_880, 5_898_240), ("w2.scale", "F8_E8M0", [5120, 72], 12_165_120, 368_640),
        ("w3.weight", "I8", [2304, 2560], 12_533_760, 5_898_240), ("w3.scale", "F8_E8M0", [2304, 160], 18_432_000, 368_640)]),
    "qwen": (2_611_200, 2560, 640, [
        ("gate_up.weight", "U32", [1280, 320], 0, 1_638_400), ("gate_up.scale", "U8", [1280, 80], 1_638_400, 102_400),
        ("down.weight", "U32", [2560, 80], 1_740_800, 819_200), ("down.scale", "U8", [2560, 20], 2_560_000, 51_200)]),
}


@pytest.mark.parametrize("model", sorted(REFERENCE_LAYOUTS))
def test_reference_region_tables_are_accepted(tmp_path, model):
    """The loader accepts the reference's own region tables, derives their shapes, and lands
    one expert's bytes in slot order (DeepSeek: w3 | w1 | w3.scale | w1.scale | w2 | w2.scale)."""
    blob, hidden, inter, regions = REFERENCE_LAYOUTS[model]
    (tmp_path / "experts").mkdir()
    rng = np.random.default_rng(len(model))
    data = rng.integers(0, 256, size=blob, dtype=np.uint8)
    (tmp_path / "experts" / "layer_00.bin").write_bytes(data.tobytes())
    manifest = {"files": [{"path": "experts/layer_00.bin", "size": blob}],
                "expertRegions": [{"name": n, "dtype": d, "shape": sh, "offset": o, "length": ln}
                                  for n, d, sh, o, ln in regions]}
    (tmp_path / "manifest.json").write_text(json.dumps(manifest))
    files = ExpertFiles(tmp_path)
    assert (files.blob, files.hidden, files.inter, files.experts, files.layers) == (blob, hidden, inter, 1, 1)
    assert files.blob == qwen_blob_bytes(hidden, inter)
    got = files.read(pinned=False).numpy()
    span = {n: data[o:o + ln] for n, _, _, o, ln in regions}
    order = (("gate_up.weight", "gate_up.scale", "down.weight", "down.scale") if model == "qwen" else
             ("w3.weight", "w1.weight", "w3.scale", "w1.scale", "w2.weight", "w2.scale"))
    assert np.array_equal(got, np.concatenate([span[n] for n in order]))
    t = files.table(files.read(pinned=False), 0)
    assert t.up_first == (model != "qwen") and (t.hidden, t.inter) == (hidden, inter)
