"""Raw tensor dumps in trellis2.c's tool formats (host code of the library).

Reading follows tools/debug/trellis_structured_latent.c:237-333 ([N,4] when
the int32 count is a multiple of 4, else [N,3] with batch 0; whole files of
floats); writing follows src/ops/sparse/cuda/forward.cu:99-223 ("%03d_<name>"
files and one "<name>\\t<rows>x<cols>\\t<dtype>\\t<file>" manifest line each).
The CPU tests call host code only; the device variants are marked gpu.
"""
import os

import numpy as np
import pytest

import sparse_hip as sh


def test_read_coords_i32_shapes(tmp_path):
    c4 = np.arange(24, dtype=np.int32).reshape(6, 4)
    p4 = tmp_path / "c4.i32"
    c4.tofile(p4)
    assert np.array_equal(sh.read_coords_i32(str(p4)), c4)
    # The same 24 values read as [N,3] when forced: batch 0 prepended.
    forced = sh.read_coords_i32(str(p4), force_xyz=True)
    assert forced.shape == (8, 4) and np.all(forced[:, 0] == 0)
    assert np.array_equal(forced[:, 1:], c4.reshape(8, 3))
    c3 = np.arange(9, dtype=np.int32).reshape(3, 3)  # 9 values: not a multiple of 4
    p3 = tmp_path / "c3.i32"
    c3.tofile(p3)
    got = sh.read_coords_i32(str(p3))
    assert got.tolist() == [[0, 0, 1, 2], [0, 3, 4, 5], [0, 6, 7, 8]]
    bad = tmp_path / "bad.i32"
    np.arange(5, dtype=np.int32).tofile(bad)  # neither [N,4] nor [N,3]
    with pytest.raises(sh.HipError) as ei:
        sh.read_coords_i32(str(bad))
    assert ei.value.status == sh.PARSE_ERROR
    with pytest.raises(sh.HipError) as ei:
        sh.read_coords_i32(str(tmp_path / "missing.i32"))
    assert ei.value.status == sh.IO_ERROR


def test_read_f32_whole_file(tmp_path):
    x = np.random.default_rng(0).standard_normal(37).astype(np.float32)
    p = tmp_path / "x.f32"
    x.tofile(p)
    assert np.array_equal(sh.read_f32(str(p)), x)
    odd = tmp_path / "odd.f32"
    odd.write_bytes(bytes(7))
    with pytest.raises(sh.HipError) as ei:
        sh.read_f32(str(odd))
    assert ei.value.status == sh.PARSE_ERROR
    empty = tmp_path / "empty.f32"
    empty.write_bytes(b"")
    assert sh.read_f32(str(empty)).size == 0


def test_dump_files_and_manifest(tmp_path):
    d = sh.Dump(str(tmp_path / "dump"), "shape_decoder_intermediates.tsv")
    coords = np.array([[0, 1, 2, 3], [0, 4, 5, 6]], np.int32)
    feats = np.arange(14, dtype=np.float32).reshape(2, 7)
    d.host("coords", coords)
    d.host("head_out", feats)
    d.close()
    root = tmp_path / "dump"
    lines = (root / "shape_decoder_intermediates.tsv").read_text().splitlines()
    assert lines == ["coords\t2x4\ti32\t000_coords.i32", "head_out\t2x7\tf32\t001_head_out.f32"]
    assert np.array_equal(np.fromfile(root / "000_coords.i32", dtype=np.int32).reshape(2, 4), coords)
    assert np.array_equal(np.fromfile(root / "001_head_out.f32", dtype=np.float32).reshape(2, 7), feats)
    # What was written reads back through the tool readers.
    assert np.array_equal(sh.read_coords_i32(str(root / "000_coords.i32")), coords)
    assert np.array_equal(sh.read_f32(str(root / "001_head_out.f32")), feats.ravel())


@pytest.mark.gpu
def test_dump_device_buffer_and_map(tmp_path):
    be = sh.Backend(0, sh.BF16)
    try:
        rng = np.random.default_rng(3)
        x = rng.standard_normal((100, 7)).astype(np.float32)
        buf = be.upload(x)
        coords = np.stack([np.zeros(100), rng.integers(0, 50, 100), rng.integers(0, 50, 100),
                           rng.integers(0, 50, 100)], axis=1).astype(np.int32)
        cmap = be.upload_coords(coords)
        d = sh.Dump(str(tmp_path / "dev"), "manifest.tsv")
        d.buffer(be, "feats", buf, 100, 7)
        d.map_coords(be, "coords", cmap)
        d.close()
        root = tmp_path / "dev"
        assert (root / "manifest.tsv").read_text().splitlines() == ["feats\t100x7\tf32\t000_feats.f32",
                                                                    "coords\t100x4\ti32\t001_coords.i32"]
        got = np.fromfile(root / "000_feats.f32", dtype=np.float32).reshape(100, 7)
        assert np.array_equal(got, be.download(buf).reshape(100, 7))
        assert np.array_equal(got, sh.storage_round(x, sh.BF16))
        assert np.array_equal(np.fromfile(root / "001_coords.i32", dtype=np.int32).reshape(100, 4), coords)
    finally:
        be.destroy()
