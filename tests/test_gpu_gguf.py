"""GPU: fkv_gguf_upload puts the GGUF data section in HBM byte for byte, every tensor at
its data_offset, and an uploaded Q8_0 tensor feeds the GEMV exactly as the file's bytes
feed the oracle (the path gguf::load -> GgufModel::tensor_bytes -> Kernels::gemv of
crates/model/src/weights.rs:15-26, on the device)."""
import numpy as np
import pytest

from oracle import ref
from tests import gguf_build as gb

pytestmark = pytest.mark.gpu


def _q8_bytes(rng, rows, cols):
    nb = rows * cols // 32
    out = np.empty((nb, 34), np.uint8)
    sc = (rng.integers(0x1400, 0x2400, nb) | (rng.integers(0, 2, nb) << 15)).astype(np.uint16)
    out[:, 0], out[:, 1] = sc & 0xff, sc >> 8
    out[:, 2:] = rng.integers(-128, 128, (nb, 32)).astype(np.int8).view(np.uint8)
    return out.reshape(-1).tobytes()


def _model(rng):
    """A file with Q8_0, F32 and F16 tensors at alignment 64, a few MB of data."""
    tensors, cursor = [], 0
    specs = [("blk.0.attn_q.weight", [256, 64], 8), ("blk.0.attn_norm.weight", [256], 0),
             ("blk.0.ffn_up.weight", [512, 96], 8), ("output_norm.weight", [100], 1),
             ("token_embd.weight", [1024, 512], 8)]
    for name, dims, gt in specs:
        off = gb.align_up(cursor, 64)
        n = int(np.prod(dims))
        if gt == 8:
            data = _q8_bytes(rng, dims[1], dims[0])
        else:
            data = rng.integers(0, 256, n * (4 if gt == 0 else 2), dtype=np.uint8).tobytes()
        tensors.append((name, dims, gt, off, data))
        cursor = off + len(data)
    kvs = [("general.alignment", gb.U32(64)), ("general.architecture", gb.Str("llama"))]
    return gb.build(3, kvs, tensors, 64)


@pytest.mark.parametrize("chunk,threads", [(0, 0), (1 << 20, 3), (4096, 1), (1000003, 8)])
def test_upload_is_the_data_section(tmp_path, chunk, threads):
    import torch
    import ferrum_amd as fa
    data = _model(np.random.default_rng(7))
    path = tmp_path / "m.gguf"
    path.write_bytes(data)
    with fa.GgufFile(str(path)) as f:
        dst = torch.full((f.data_bytes + 100,), 0xEE, dtype=torch.uint8, device="cuda")
        f.upload(dst, chunk_bytes=chunk, threads=threads)
        torch.cuda.synchronize()
        got = dst.cpu().numpy()
        section = np.frombuffer(data, np.uint8)[f.data_start:]
        assert np.array_equal(got[:f.data_bytes], section)
        assert np.all(got[f.data_bytes:] == 0xEE)          # nothing past the section
        for t in f.tensors:
            start = f.data_start + t.data_offset
            assert np.array_equal(f.device_tensor(dst, t.name).cpu().numpy(),
                                  np.frombuffer(data, np.uint8)[start:start + t.nbytes])


def test_uploaded_q8_tensor_feeds_the_gemv(tmp_path):
    import torch
    import ferrum_amd as fa
    rng = np.random.default_rng(9)
    data = _model(rng)
    path = tmp_path / "m.gguf"
    path.write_bytes(data)
    with fa.GgufFile(str(path)) as f:
        dst = torch.empty(f.data_bytes, dtype=torch.uint8, device="cuda")
        f.upload(dst)
        for name in ("blk.0.attn_q.weight", "blk.0.ffn_up.weight", "token_embd.weight"):
            t = f.tensor(name)
            cols, rows = t.shape                            # GGUF [ne0 = cols, ne1 = rows]
            x = rng.standard_normal((2, cols)).astype(np.float32)
            y = torch.empty(2, rows, dtype=torch.float32, device="cuda")
            fa.gemm_q8_0(f.device_tensor(dst, name), rows, cols, torch.from_numpy(x).cuda(), 2, y)
            torch.cuda.synchronize()
            start = f.data_start + t.data_offset
            w = np.frombuffer(data, np.uint8)[start:start + t.nbytes]
            want = ref.q8_gemm(w, rows, cols, x)
            assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32)), name


def test_upload_rejects_a_short_buffer(tmp_path):
    import torch
    import ferrum_amd as fa
    path = tmp_path / "m.gguf"
    path.write_bytes(_model(np.random.default_rng(1)))
    with fa.GgufFile(str(path)) as f:
        dst = torch.zeros(f.data_bytes - 1, dtype=torch.uint8, device="cuda")
        with pytest.raises(fa.InvalidRequest, match="^device buffer smaller than the data section$"):
            f.upload(dst)
        torch.cuda.synchronize()
        assert int(dst.count_nonzero()) == 0


def test_upload_reports_a_file_cut_short_after_open(tmp_path):
    # the directory was decoded at open; the data section is read at upload, so a file that
    # shrinks in between is a read error, not a crash
    import os
    import torch
    import ferrum_amd as fa
    path = tmp_path / "m.gguf"
    path.write_bytes(_model(np.random.default_rng(3)))
    with fa.GgufFile(str(path)) as f:
        dst = torch.zeros(f.data_bytes, dtype=torch.uint8, device="cuda")
        os.truncate(path, f.data_start + f.data_bytes // 2)
        with pytest.raises(fa.GgufError, match=r"^gguf: failed to read tensor data: .*\(os error 5\)$"):
            f.upload(dst, chunk_bytes=1 << 16, threads=4)
        torch.cuda.synchronize()


def test_upload_past_four_gib(tmp_path):
    # a sparse 5 GiB F32 tensor: offsets beyond 32 bits in the file, the staging and HBM
    import torch
    import ferrum_amd as fa
    n = (5 << 30) // 4
    hdr = gb.build(3, [], [("big", [n], 0, 0, b"")], 32)
    marks = {0: b"head", (4 << 30) - 3: b"edge", (4 << 30) + 12345: b"past", n * 4 - 4: b"tail"}
    path = tmp_path / "big.gguf"
    with open(path, "wb") as f:
        f.write(hdr)
        f.truncate(len(hdr) + n * 4)
        for off, m in marks.items():
            f.seek(len(hdr) + off)
            f.write(m)
    with fa.GgufFile(str(path)) as g:
        assert g.data_bytes == n * 4 and g.tensor("big").nbytes == n * 4
        dst = torch.full((n * 4,), 0x5A, dtype=torch.uint8, device="cuda")
        g.upload(dst)
        torch.cuda.synchronize()
        for off, m in marks.items():
            assert bytes(dst[off:off + 4].cpu().numpy()) == m, off
        # everything else is the file's zeros: the sum is the marks' bytes alone
        assert int(dst.sum(dtype=torch.int64)) == sum(sum(m) for m in marks.values())
