"""CPU checks of the expert-file layer (fm_expert_io.h): mode detection, tiered
manifest parsing and validation, offset lookup and byte-exact parallel preads.
Files are written in the reference's on-disk format (repack_experts_tiered.py:
345-425); the 397B manifest case uses the reference's hot-expert sets
(tests/golden/tiered_397b_hot.json, made by make_tiered_397b.py).  No GPU."""
import json
import os

import numpy as np
import pytest

import fmoe_amd as fm
from fmoe_amd import synth
from fmoe_amd.expert_io import STORE_2BIT, STORE_4BIT, STORE_AUTO, STORE_TIERED, ExpertStore, write_layer_files

H, I = 512, 256  # small experts: 4-bit 221,184 B, 2-bit 122,880 B
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def sizes(h=H, i=I):
    return fm.layout_of(h, i, 64, 4).size, fm.layout_of(h, i, 64, 2).size


def model(nl, ne, bits_of, h=H, i=I, seed=0):
    return [[(synth.expert_blob((seed, l, e), h, i, bits_of(l, e)), bits_of(l, e)) for e in range(ne)]
            for l in range(nl)]


@pytest.fixture
def three_formats(tmp_path):
    s4, s2 = sizes()
    m4 = model(2, 6, lambda l, e: 4, seed=1)
    m2 = model(2, 6, lambda l, e: 2, seed=2)
    mt = model(2, 6, lambda l, e: 4 if (e + l) % 3 == 0 else 2, seed=3)
    write_layer_files(tmp_path, m4, "4bit", s4, s2)
    write_layer_files(tmp_path, m2, "2bit", s4, s2)
    man = write_layer_files(tmp_path, mt, "tiered", s4, s2, threshold=0.25)
    return tmp_path, m4, m2, mt, man


def test_layout_sizes_match_reference_constants():
    # config.h:94-137 at the 397B/35B dimensions
    assert sizes(4096, 1024) == (7077888, 3932160)


def test_auto_detection_order(three_formats):
    d, *_ = three_formats
    with ExpertStore(d, 2, 6, H, I) as s:
        assert s.info().mode == STORE_TIERED  # manifest wins (generate.h:1813-1822)
    os.rename(d / "packed_experts_tiered" / "tiered_manifest.json", d / "m.json")
    with ExpertStore(d, 2, 6, H, I) as s:
        assert s.info().mode == STORE_4BIT  # 4-bit present: 2-bit not auto-selected
    os.rename(d / "packed_experts", d / "p4")
    with ExpertStore(d, 2, 6, H, I) as s:
        assert s.info().mode == STORE_2BIT  # only 2-bit files (generate.h:1832-1846)
    os.rename(d / "packed_experts_2bit", d / "p2")
    with ExpertStore(d, 2, 6, H, I) as s:
        i = s.info()
        assert i.mode == STORE_4BIT and i.layers_available == 0


@pytest.mark.parametrize("mode", [STORE_4BIT, STORE_2BIT, STORE_TIERED])
def test_extents_and_bytes(three_formats, mode):
    d, m4, m2, mt, man = three_formats
    m = {STORE_4BIT: m4, STORE_2BIT: m2, STORE_TIERED: mt}[mode]
    s4, s2 = sizes()
    with ExpertStore(d, 2, 6, H, I, mode=mode, io_threads=3) as s:
        info = s.info()
        assert (info.expert_size_4bit, info.expert_size_2bit) == (s4, s2)
        assert info.layers_available == 2 and info.manifest_warnings == 0
        for l in range(2):
            off = 0
            for e in range(6):
                o, sz, b = s.extent(l, e)
                assert b == m[l][e][1] and sz == m[l][e][0].size and o == off  # timing.h:138-148
                if mode == STORE_TIERED:
                    assert man["layers"][str(l)]["experts"][e] == {"offset": o, "size": sz, "bits": b}
                off += sz
            assert s.layer_bytes(l) == off
        ids = [5, 0, 3, 3, 1]
        blobs, valid = s.read(1, ids)
        assert valid == [1] * len(ids)
        for b, e in zip(blobs, ids):
            assert np.array_equal(b, m[1][e][0])


def test_multi_chunk_reads_are_exact(tmp_path):
    """Full-size 4-bit experts (7 MB) are split into page-aligned chunks over the workers."""
    s4, s2 = sizes(4096, 1024)
    m = model(1, 3, lambda l, e: 4 if e != 1 else 2, h=4096, i=1024, seed=7)
    write_layer_files(tmp_path, m, "tiered", s4, s2)
    with ExpertStore(tmp_path, 1, 3, 4096, 1024, io_threads=8) as s:
        blobs, valid = s.read(0, [2, 1, 0])
        assert valid == [1, 1, 1]
        for b, e in zip(blobs, [2, 1, 0]):
            assert np.array_equal(b, m[0][e][0])


def test_manifest_validation(three_formats):
    d, *_ = three_formats
    mp = d / "packed_experts_tiered" / "tiered_manifest.json"
    man = json.loads(mp.read_text())

    def reopen(mutate, **kw):
        m = json.loads(json.dumps(man))
        mutate(m)
        mp.write_text(json.dumps(m))
        return ExpertStore(d, 2, 6, H, I, mode=STORE_TIERED, **kw)

    # num_layers / num_experts / expert sizes must match (config.h:335-355)
    for mut in (lambda m: m.update(num_layers=3), lambda m: m.update(num_experts=7),
                lambda m: m.update(expert_size_4bit=123), lambda m: m.update(expert_size_2bit=99)):
        with pytest.raises(fm.FmError) as ei:
            reopen(mut)
        assert ei.value.code == -1  # FM_ERR_INVALID
    # absent expert sizes are not checked
    s = reopen(lambda m: (m.pop("expert_size_4bit"), m.pop("expert_size_2bit")))
    assert s.info().manifest_warnings == 0
    s.close()
    # missing layer -> 4-bit sequential defaults, one warning (config.h:361-369)
    s = reopen(lambda m: m["layers"].pop("1"))
    assert s.info().manifest_warnings == 1
    s4, _ = sizes()
    assert [s.extent(1, e) for e in range(6)] == [(e * s4, s4, 4) for e in range(6)]
    s.close()
    # invalid bits -> treated as 4-bit, one warning (config.h:375-380); offsets/sizes kept
    s = reopen(lambda m: m["layers"]["0"]["experts"][2].update(bits=3))
    assert s.info().manifest_warnings == 1
    assert s.extent(0, 2)[2] == 4 and s.extent(0, 2)[:2] == (man["layers"]["0"]["experts"][2]["offset"],
                                                              man["layers"]["0"]["experts"][2]["size"])
    s.close()
    # short expert list -> empty entries (calloc'd in the reference): warning, reads invalid
    s = reopen(lambda m: m["layers"]["0"].update(experts=m["layers"]["0"]["experts"][:4]))
    assert s.info().manifest_warnings == 2
    assert s.extent(0, 5) == (0, 0, 0)
    _, valid = s.read(0, [0, 5])
    assert valid == [1, 0]
    s.close()
    # malformed JSON
    mp.write_text('{"num_layers": 2, "num_experts": ')
    with pytest.raises(fm.FmError):
        ExpertStore(d, 2, 6, H, I, mode=STORE_TIERED)
    # explicit tiered with no manifest
    mp.unlink()
    with pytest.raises(fm.FmError):
        ExpertStore(d, 2, 6, H, I, mode=STORE_TIERED)


def test_missing_and_truncated_files(three_formats):
    d, m4, *_ = three_formats
    os.remove(d / "packed_experts" / "layer_01.bin")
    f0 = d / "packed_experts" / "layer_00.bin"
    os.truncate(f0, f0.stat().st_size - 100)
    with ExpertStore(d, 2, 6, H, I, mode=STORE_4BIT) as s:
        assert s.info().layers_available == 1
        blobs, valid = s.read(0, [0, 5, 4])
        assert valid == [1, 0, 1]  # the last expert is 100 bytes short
        assert np.array_equal(blobs[0], m4[0][0][0]) and np.array_equal(blobs[2], m4[0][4][0])
        _, valid = s.read(1, [0, 1])
        assert valid == [0, 0]


def test_argument_errors(three_formats):
    d, *_ = three_formats
    with ExpertStore(d, 2, 6, H, I) as s:
        for bad in ((2, 0), (-1, 0), (0, 6), (0, -1)):
            with pytest.raises(fm.FmError):
                s.extent(*bad)
        with pytest.raises(fm.FmError):
            s.read(0, [0, 9])
        with pytest.raises(fm.FmError):
            s.layer_bytes(5)
    with pytest.raises(fm.FmError):
        ExpertStore(d, 0, 6, H, I)
    with pytest.raises(fm.FmError):
        ExpertStore(d, 2, 6, H, I, mode=7)
    with pytest.raises(fm.FmError):
        ExpertStore(d, 2, 6, 500, I)  # hidden not a multiple of the group size


def test_397b_tiered_manifest(tmp_path):
    """The 397B model's hot sets (reference hot_experts_397B.json): a 60 x 512 manifest
    built the way repack_experts_tiered.py:376-400 builds it (hot -> 4-bit, others
    2-bit, blobs back to back in expert order) parses to the same extents."""
    hot = json.load(open(os.path.join(GOLDEN, "tiered_397b_hot.json")))
    L, E = hot["num_layers"], hot["num_experts"]
    s4, s2 = 7077888, 3932160
    layers = {}
    expect = np.zeros((L, E, 3), np.int64)
    for l in range(L):
        hs = set(hot["hot_experts"][str(l)])
        off, ents = 0, []
        for e in range(E):
            b, sz = (4, s4) if e in hs else (2, s2)
            ents.append({"offset": off, "size": sz, "bits": b})
            expect[l, e] = (off, sz, b)
            off += sz
        layers[str(l)] = {"experts": ents, "file_size": off}
    d = tmp_path / "packed_experts_tiered"
    d.mkdir()
    (d / "tiered_manifest.json").write_text(json.dumps(
        {"expert_size_4bit": s4, "expert_size_2bit": s2, "num_layers": L, "num_experts": E,
         "threshold": hot["threshold"], "gptq_source": None, "layers": layers}, indent=2))
    with ExpertStore(tmp_path, L, E, 4096, 1024) as s:
        info = s.info()
        assert info.mode == STORE_TIERED and info.layers_available == 0 and info.manifest_warnings == 0
        got = np.array([[s.extent(l, e) for e in range(E)] for l in range(L)], np.int64)
        assert np.array_equal(got, expect)
        assert int((got[:, :, 2] == 4).sum()) == hot["total_hot"] == 7680
        assert int((got[:, :, 2] == 2).sum()) == hot["total_cold"] == 23040
        # 128 hot + 384 cold per layer: 128 * 7,077,888 + 384 * 3,932,160
        assert all(s.layer_bytes(l) == 2415919104 for l in range(L))
        # layer files absent: every read reports invalid, nothing raises
        _, valid = s.read(3, [0, 1, 511])
        assert valid == [0, 0, 0]
