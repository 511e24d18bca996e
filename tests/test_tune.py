"""The GEMV-vs-tile tuning table and its text store (host side, no GPU)."""
import pytest

from brain_amd._lib import BrainHipError, check, load

GEMV, TILE = 2, 1  # BH_VARIANT_WORKGROUP_PER_OUTPUT, BH_VARIANT_PACKED_INT8


def test_buckets_and_store(tmp_path):
    L = load()
    L.bh_tune_clear()
    check(L.bh_tune_set(3, 3072, 1024, TILE))          # bucket 4
    assert L.bh_tune_get(4, 3072, 1024) == TILE
    assert L.bh_tune_get(3, 3072, 1024) == TILE
    assert L.bh_tune_get(2, 3072, 1024) == 0           # bucket 2: nothing recorded
    assert L.bh_tune_get(5, 3072, 1024) == 0           # bucket 8
    assert L.bh_tune_get(64, 3072, 1024) == 0          # above the decode regime
    check(L.bh_tune_set(32, 151936, 1024, GEMV))
    p = str(tmp_path / "tune.txt")
    check(L.bh_tune_save(p.encode()))
    L.bh_tune_clear()
    assert L.bh_tune_get(4, 3072, 1024) == 0
    assert check(L.bh_tune_load(p.encode())) == 2
    assert L.bh_tune_get(4, 3072, 1024) == TILE and L.bh_tune_get(17, 151936, 1024) == GEMV
    check(L.bh_tune_set(4, 3072, 1024, 0))             # remove
    assert L.bh_tune_get(4, 3072, 1024) == 0
    L.bh_tune_clear()


def test_store_rejects_foreign_files(tmp_path):
    L = load()
    p = tmp_path / "t.txt"
    p.write_text("something else\n1 2 3 1\n")
    with pytest.raises(BrainHipError):
        check(L.bh_tune_load(str(p).encode()))
    good = tmp_path / "g.txt"
    check(L.bh_tune_save(str(good).encode()))
    good.write_text(good.read_text() + "1 2 3 9\n")
    with pytest.raises(BrainHipError):
        check(L.bh_tune_load(str(good).encode()))
    with pytest.raises(BrainHipError):
        check(L.bh_tune_set(0, 1, 4, TILE))
    with pytest.raises(BrainHipError):
        check(L.bh_tune_set(4, 1, 4, 7))


def test_store_is_keyed_by_device_and_kernel_build(tmp_path):
    """A table measured on another device or another GEMV/GEMM build does not
    load (crates/qwen3/src/serve.rs:1118-1121 keys by adapter + kernel source)."""
    from brain_amd import build as hipbuild
    L = load()
    L.bh_tune_clear()
    check(L.bh_tune_set(4, 3072, 1024, TILE))
    p = tmp_path / "tune.txt"
    check(L.bh_tune_save(str(p).encode()))
    header, *rest = p.read_text().splitlines()
    fields = header.split()
    assert fields[:5] == ["brain-hip-tune", "2", "abi", str(L.bh_abi_version()), "device"]
    assert fields[6] == "kernels" and int(fields[7], 16) == hipbuild.kernel_fingerprint()
    L.bh_tune_clear()
    assert check(L.bh_tune_load(str(p).encode())) == 1          # own table loads
    for i, foreign in ((5, "gfx942|AMD_Instinct_MI300X"), (7, "%016x" % (hipbuild.kernel_fingerprint() ^ 1))):
        f = list(fields)
        f[i] = foreign
        q = tmp_path / f"foreign{i}.txt"
        q.write_text(" ".join(f) + "\n" + "\n".join(rest) + "\n")
        L.bh_tune_clear()
        with pytest.raises(BrainHipError, match="another device or kernel build"):
            check(L.bh_tune_load(str(q).encode()))
        assert L.bh_tune_get(4, 3072, 1024) == 0
    L.bh_tune_clear()
