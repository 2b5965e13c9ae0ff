"""Host-side reading of the reference's session files (DS4CUDAK,
cuda/kv_persist.cuh): ds4hip_ds4cudak_probe returns the header fields and
per-layer counts of a file written in the reference's layout, and refuses
wrong magic, wrong geometry, a wrong payload size, truncation and trailing
bytes."""
import numpy as np
import pytest

from ds4cuda_amd import Ds4HipError
from ds4cuda_amd.session import probe_ds4cudak
import ds4cudak_file as F


@pytest.fixture(scope="module")
def ref_file(tmp_path_factory):
    p = tmp_path_factory.mktemp("kvc") / "ref.kvc"
    layers = {0: {"n_raw": 128}, 1: {"n_raw": 128}, 2: {"n_raw": 128, "n_comp": 50, "n_idx": 50},
              3: {"n_raw": 128, "n_comp": 1}}
    for il in range(4, 43):
        layers[il] = {"n_raw": 128, "n_comp": 50 if il % 2 == 0 else 1, "n_idx": 50 if il % 2 == 0 else 0}
    F.write(p, 256, 203, 203, range(1000, 1100), layers)
    return p


def test_probe_reads_header_and_counts(ref_file):
    info = probe_ds4cudak(ref_file)
    assert (info.max_context, info.pos, info.n_tokens_processed, info.cap_raw) == (256, 203, 203, 128)
    assert info.n_prompt_tokens == 64 and list(info.prompt_token_ids) == list(range(1000, 1064))
    assert list(info.n_raw) == [128] * 43
    assert info.n_comp[2] == 50 and info.n_comp[3] == 1 and info.n_comp[0] == 0
    assert info.n_index_comp[2] == 50 and info.n_index_comp[3] == 0
    assert info.file_bytes == ref_file.stat().st_size


def expect_refused(path, code):
    with pytest.raises(Ds4HipError) as e:
        probe_ds4cudak(path)
    assert e.value.code == code


def test_probe_refuses_bad_files(ref_file, tmp_path):
    data = ref_file.read_bytes()
    bad = tmp_path / "bad.kvc"
    bad.write_bytes(b"XS4CUDAK" + data[8:])
    expect_refused(bad, -22)                                  # magic
    bad.write_bytes(data[:8] + (2).to_bytes(4, "little") + data[12:])
    expect_refused(bad, -22)                                  # version
    bad.write_bytes(data[:32] + (64).to_bytes(4, "little") + data[36:])
    expect_refused(bad, -22)                                  # cap_raw against max_context
    meta0 = 360
    bad.write_bytes(data[:meta0 + 32] + (1).to_bytes(8, "little") + data[meta0 + 40:])
    expect_refused(bad, -22)                                  # layer 0 payload size
    bad.write_bytes(data[:meta0 + 20] + (129).to_bytes(4, "little") + data[meta0 + 24:])
    expect_refused(bad, -22)                                  # n_raw above cap_raw
    bad.write_bytes(data[:-8] + b"DS4CUDA2")
    expect_refused(bad, -22)                                  # trailer
    bad.write_bytes(data + b"\0")
    expect_refused(bad, -22)                                  # bytes after the trailer
    bad.write_bytes(data[: len(data) // 2])
    expect_refused(bad, -5)                                   # truncated
    expect_refused(tmp_path / "missing.kvc", -5)
