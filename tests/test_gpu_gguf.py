"""GGUF file -> HBM -> GEMV: the uploaded data section is byte-identical to
the file's, and every quantised tensor, used through its TensorStorage view
(encodeProjection dispatch on data type and GGUF shape [K, M]), gives the
same outputs as the same bytes passed to the format's own GEMV entry, and
matches the CPU oracle (relative L2 <= 1e-3)."""
import hashlib

import numpy as np
import pytest

import edgerunner_amd.synth as synth
from edgerunner_amd import GEMVKernel
from edgerunner_amd.gguf import GGUFLoader, GGUFMetadataValueType as VT, GGUFTensorType as TT, write_gguf
from oracle import ref
from conftest import rel_l2

pytestmark = pytest.mark.gpu

# (name, GGUF type, M rows, K columns, synth format)
TENSORS = [("blk.0.attn_q.weight", TT.q4_K, 2048, 1024, "q4_k"),
           ("blk.0.ffn_down.weight", TT.q6_K, 1024, 3072, "q6_k"),
           ("blk.0.attn_v.weight", TT.q8_0, 3072, 1024, "q8_0"),
           ("output.weight", TT.q6_K, 4096, 1024, "q6_k")]
DSCALE = {"q8_0": {"dscale": 0.02}, "q4_k": {"dscale": 0.01, "dminscale": 0.01},
          "q6_k": {"dscale": 0.005}}


def model_file(tmp_path, alignment=32):
    tensors, raw = [], {}
    for t, (name, tt, M, K, fmt) in enumerate(TENSORS):
        W = synth.weights(fmt, synth.seed(60, t), M, K, **DSCALE[fmt])
        raw[name] = W
        tensors.append((name, [K, M], tt, W.tobytes()))
    norm = synth.normal_f32(synth.seed(60, 9), 1024)
    tensors.append(("blk.0.attn_norm.weight", [1024], TT.f32, norm.tobytes()))
    md = [("general.architecture", VT.string, "qwen3"), ("qwen3.block_count", VT.uint32, 1)]
    if alignment != 32:
        md.append(("general.alignment", VT.uint32, alignment))
    p = write_gguf(tmp_path / f"model_{alignment}.gguf", md, tensors, alignment=alignment)
    return p, raw


@pytest.mark.parametrize("alignment", [32, 4096])
def test_gguf_to_hbm_to_gemv(ctx, tmp_path, alignment):
    path, raw = model_file(tmp_path, alignment)
    loader = GGUFLoader(path)
    weights = loader.load(ctx)
    off, n = loader.dataSection()
    dev = loader.deviceData.download(np.uint8)
    assert dev.size == n
    assert hashlib.sha256(dev.tobytes()).digest() == hashlib.sha256(path.read_bytes()[off:]).digest()
    gemv = GEMVKernel(ctx)
    for t, (name, tt, M, K, fmt) in enumerate(TENSORS):
        ts = weights[name]
        assert ts.dataType == tt.tensorDataType and ts.shape == (K, M)
        x = synth.normal_f32(synth.seed(60, 20 + t), K)
        xb, yb = ctx.upload(x), ctx.alloc(4 * M)
        gemv.encodeTensor(None, ts, xb, yb)
        ctx.synchronize()
        y = yb.download(np.float32)
        xb.free()
        yb.free()
        direct = {"q4_k": gemv.executeQ4KWeights, "q6_k": gemv.executeQ6KWeights,
                  "q8_0": gemv.executeQ8_0Weights}[fmt](raw[name], x, M, K)
        assert np.array_equal(y, direct), name
        assert rel_l2(y, ref.gemv(fmt, raw[name], x, M, K, threads=ref.max_threads())) < 1e-3, name
    norm = weights["blk.0.attn_norm.weight"]
    assert np.array_equal(norm.buffer.download(np.float32), synth.normal_f32(synth.seed(60, 9), 1024))
    loader.close()


def test_large_upload_is_byte_exact(ctx, tmp_path):
    """A data section spanning several staging chunks (and a partial last one)."""
    rng = np.random.default_rng(61)
    payload = rng.integers(0, 256, size=(150 << 20) + 4321, dtype=np.uint8)
    p = write_gguf(tmp_path / "big.gguf", [("general.architecture", VT.string, "llama")],
                   [("blob", [payload.size], TT.i8, payload.tobytes())])
    loader = GGUFLoader(p)
    weights = loader.load(ctx)
    got = weights["blob"].buffer.download(np.uint8)
    assert np.array_equal(got, payload)
    loader.close()
