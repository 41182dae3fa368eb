"""Checkpoint formats through the C++ API: the AdamParameter record stream
(AdamParameter::save/load, Engine/engine.cu:139-268) and TEMB embedding files
(TextualEmbedding::save/load/load_replace, Engine/transformer.cu:246-484).
Files are parsed here byte by byte, so the layout itself is pinned, not only
the round trip."""
import struct

import numpy as np
import pytest

from ml_engine_amd.configs import BlockConfig, MLPConfig, block_data, mlp_data
from ml_engine_amd.models import STEP_ALL, Model

pytestmark = pytest.mark.gpu


def parse_adam_records(raw: bytes):
    """[u32 name_len][name][i32 total][f32 W][f32 m][f32 v] per parameter."""
    out, o = [], 0
    while o < len(raw):
        (nl,) = struct.unpack_from("<I", raw, o)
        o += 4
        name = raw[o:o + nl].decode()
        o += nl
        (total,) = struct.unpack_from("<i", raw, o)
        o += 4
        arrs = []
        for _ in range(3):
            arrs.append(np.frombuffer(raw, np.float32, total, o).copy())
            o += 4 * total
        out.append((name, total, *arrs))
    return out


def test_adam_checkpoint_layout_and_round_trip(hip, tmp_path):
    cfg = MLPConfig()
    x, labels, params = mlp_data(cfg, seed=0)
    m = Model("mlp", cfg.dims())
    for i, p in enumerate(params):
        m.set(i, p)
    m.input(0, x)
    m.input(1, labels)
    for _ in range(2):  # non-zero moments
        m.step(cfg.lr, STEP_ALL)
    m.sync()
    path = tmp_path / "mlp.ckpt"
    m.save(path)
    recs = parse_adam_records(path.read_bytes())
    assert [r[0] for r in recs] == m.names
    for i, (name, total, w, mm, vv) in enumerate(recs):
        assert total == m.numel[i]
        np.testing.assert_array_equal(w, m.get(i, 0))
        np.testing.assert_array_equal(mm, m.get(i, 2))
        np.testing.assert_array_equal(vv, m.get(i, 3))
        assert np.any(mm != 0) and np.any(vv != 0)
    fresh = Model("mlp", cfg.dims(), seed=11)
    assert not np.array_equal(fresh.get(0, 0), m.get(0, 0))
    fresh.load(path)
    for i in range(len(m.names)):
        for which in (0, 2, 3):
            np.testing.assert_array_equal(fresh.get(i, which), m.get(i, which))
        assert fresh.t(i) == 1  # the step counter is not part of the record, as in the reference
    fresh.close()
    m.close()


def parse_temb(raw: bytes):
    magic, version, dim, n = struct.unpack_from("<IIii", raw, 0)
    o = 16
    words = {}
    for _ in range(n):
        (wl,) = struct.unpack_from("<I", raw, o)
        o += 4
        w = raw[o:o + wl].decode()
        o += wl
        (idx,) = struct.unpack_from("<i", raw, o)
        o += 4
        words[w] = idx
    table = np.frombuffer(raw, np.float32, n * dim, o).reshape(n, dim).copy()
    assert o + 4 * n * dim == len(raw)
    return magic, version, dim, words, table


def block_model(seed):
    cfg = BlockConfig(batch=2, seq=8, d_model=32, heads=2, ffn=64, vocab=50)
    _, _, params = block_data(cfg, seed=seed)
    m = Model("block", cfg.dims())
    for i, p in enumerate(params):
        m.set(i, p)
    m.sync()
    return cfg, m


def test_temb_save_load_and_replace(hip, tmp_path):
    cfg, m = block_model(3)
    E = m.get(0, 0).reshape(cfg.vocab, cfg.d_model)
    n = 40  # the vocabulary uses the first 40 of the table's 50 rows
    words = [f"w{i}" for i in range(n)]
    path = tmp_path / "emb.temb"
    m.temb_save(path, words)
    magic, version, dim, saved_words, table = parse_temb(path.read_bytes())
    assert (magic, version, dim) == (0x54454D42, 1, cfg.d_model)
    assert saved_words == {w: i for i, w in enumerate(words)}
    np.testing.assert_array_equal(table, E[:n])

    _, full = block_model(5)
    E_other = full.get(0, 0).reshape(cfg.vocab, cfg.d_model)
    assert full.temb_load(path) == n
    E_loaded = full.get(0, 0).reshape(cfg.vocab, cfg.d_model)
    np.testing.assert_array_equal(E_loaded[:n], E[:n])
    np.testing.assert_array_equal(E_loaded[n:], E_other[n:])  # rows past the vocabulary stay
    full.close()

    _, part = block_model(7)
    E_before = part.get(0, 0).reshape(cfg.vocab, cfg.d_model).copy()
    # local vocabulary: row 0 <- "w5", row 1 <- "w3", row 2 unknown word, row 3 <- "w39"
    local = ["w5", "w3", "zzz", "w39"]
    assert part.temb_load(path, replace=True, words=local) == 3
    E_after = part.get(0, 0).reshape(cfg.vocab, cfg.d_model)
    np.testing.assert_array_equal(E_after[0], E[5])
    np.testing.assert_array_equal(E_after[1], E[3])
    np.testing.assert_array_equal(E_after[2], E_before[2])
    np.testing.assert_array_equal(E_after[3], E[39])
    np.testing.assert_array_equal(E_after[4:], E_before[4:])
    part.close()
    m.close()


def test_temb_rejects_bad_files(hip, tmp_path):
    cfg, m = block_model(3)
    bad = tmp_path / "bad.temb"
    bad.write_bytes(struct.pack("<IIii", 0x12345678, 1, cfg.d_model, 0))
    assert m.temb_load(bad) == -1
    wrong_dim = tmp_path / "dim.temb"
    wrong_dim.write_bytes(struct.pack("<IIii", 0x54454D42, 1, cfg.d_model + 1, 0))
    assert m.temb_load(wrong_dim) == -1
    assert m.temb_load(tmp_path / "missing.temb", replace=True, words=["w0"]) == -1
    m.close()
