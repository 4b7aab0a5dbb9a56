"""Host-side logic of the package (no GPU): per-layer budget allocation and the
lazy safetensors reader."""
import numpy as np
import pytest
import torch

from fathom_amd import capsio
from fathom_amd.klt import allocate
from oracle import fathom_oracle as O


@pytest.mark.parametrize("seed", range(5))
def test_allocate_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    budgets = (24, 32, 40, 48, 64, 80, 96, 128)            # scripts/l4_final_alloc.py:18
    nl = 36
    err = {B: list(rng.random(nl) / (1 + i) ** rng.uniform(0.5, 2)) for i, B in enumerate(budgets)}
    for target in (32, 40, 48, 64, 80):
        got = allocate({B: dict(enumerate(v)) for B, v in err.items()}, budgets, target)
        assert [got[L] for L in range(nl)] == O.allocate(err, budgets, target)
        assert sum(got.values()) / nl >= target or all(b == budgets[-1] for b in got.values())


def test_capsio_reads_slices(tmp_path):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(0)
    t = {"k0": torch.randn(8, 300, 128, generator=g).to(torch.bfloat16),
         "q0": torch.randn(32, 300, 128, generator=g).to(torch.float16),
         "v3": torch.randn(5, 7, generator=g), "ids": torch.arange(11, dtype=torch.int64)}
    path = str(tmp_path / "caps_test.safetensors")
    save_file(t, path, metadata={"model": "synthetic"})
    f = capsio.safe_open(path, "pt")
    assert sorted(f.keys()) == sorted(t) and "k0" in f and len(f) == 4
    assert f.get_slice("q0").get_shape() == [32, 300, 128]
    assert torch.equal(f.get_slice("k0")[2], t["k0"][2])
    assert torch.equal(f.get_slice("q0")[4:12, 290:], t["q0"][4:12, 290:])
    assert torch.equal(f.get_slice("k0")[-1], t["k0"][-1])
    assert torch.equal(f["v3"], t["v3"]) and torch.equal(f.get_tensor("ids"), t["ids"])
    assert f.get_slice("k0")[3:3].shape == (0, 300, 128)
    assert torch.equal(f.get_slice("q0")[30:], t["q0"][30:]) and torch.equal(f.get_slice("v3")[..., 2], t["v3"][..., 2])
    assert torch.equal(f.get_slice("ids")[1:9:3], t["ids"][1:9:3])
    assert f.metadata_dict() == {"model": "synthetic"}
    f.close()


def test_capsio_rejects_malformed_headers(tmp_path):
    import json
    import struct
    from safetensors.torch import save_file
    path = tmp_path / "x.safetensors"
    save_file({"a": torch.zeros(4, 3)}, str(path))
    raw = path.read_bytes()
    hlen = struct.unpack("<Q", raw[:8])[0]
    hdr = json.loads(raw[8:8 + hlen])

    def write(h, body):
        b = json.dumps(h).encode()
        path.write_bytes(struct.pack("<Q", len(b)) + b + body)

    body = raw[8 + hlen:]
    write(dict(hdr, a=dict(hdr["a"], data_offsets=[0, 64])), body)      # range past the file
    with pytest.raises(ValueError):
        capsio.safe_open(str(path))
    write(dict(hdr, a=dict(hdr["a"], shape=[4, 4])), body)              # bytes != shape * dtype
    with pytest.raises(ValueError):
        capsio.safe_open(str(path))
    write(dict(hdr, a=dict(hdr["a"], dtype="C64")), body)               # unknown dtype
    with pytest.raises(ValueError):
        capsio.safe_open(str(path))
    path.write_bytes(struct.pack("<Q", 1 << 40))                        # header longer than the file
    with pytest.raises(ValueError):
        capsio.safe_open(str(path))


def test_chunk_bounds():
    from fathom_amd.offload import chunk_bounds
    assert chunk_bounds(1000, 4) == [(0, 192), (192, 448), (448, 704), (704, 1000)]
    assert chunk_bounds(16384, 4) == [(0, 4096), (4096, 8192), (8192, 12288), (12288, 16384)]
    assert chunk_bounds(100, 4) == [(0, 64), (64, 100)]          # empty chunks dropped
    assert chunk_bounds(50, 3) == [(0, 50)]
    for nblk in (1, 63, 64, 65, 777, 4097):
        for parts in (1, 2, 3, 8):
            ch = chunk_bounds(nblk, parts)
            assert ch[0][0] == 0 and ch[-1][1] == nblk and len(ch) <= parts
            assert all(a < b for a, b in ch) and all(ch[i][1] == ch[i + 1][0] for i in range(len(ch) - 1))
            assert all(b % 64 == 0 for _, b in ch[:-1])
