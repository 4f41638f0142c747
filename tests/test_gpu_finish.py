"""qlin_gemm_finish on the GPU through the C ABI: the fused bias + ReLU /
tanh-GeLU finish equals the oracle's finish applied to the stored GEMM
result (reference ops/linear.cpp:71-93, ops/cuda/quantization.cpp:465-478),
bit for bit, in every kernel family (skinny, split-K, tiled, 32x32 tiled,
packed weights), for bf16 and f16 outputs."""
import numpy as np
import pytest
import torch

from tests.test_gpu_gemm import dev_f32, dev_u8, gpu_gemm, operands, out_bits

pytestmark = pytest.mark.gpu
I8, FP8, BF16, F16 = 4, 3, 0, 5


def run_finish(dev, xq, sx, wq, sw, fmt, bias, act, path=None, out_dtype=torch.bfloat16,
               group=0, packed=False):
    from breeze_tts_cpp_amd import qlinear
    w = qlinear.pack_weights(dev_u8(wq, dev)) if packed else dev_u8(wq, dev)
    bd = None if bias is None else torch.from_numpy(bias.view(np.int16)).view(out_dtype).to(dev)
    y = qlinear.gemm_finish(dev_u8(xq, dev), dev_f32(sx, dev), w, dev_f32(sw, dev), fmt, bias=bd,
                            activation=act, out_dtype=out_dtype, input_group=group,
                            weight_group=group, path=path)
    torch.cuda.synchronize()
    return out_bits(y)


def paths():
    from breeze_tts_cpp_amd.qlinear import Path, KIND_SKINNY, KIND_TILED
    return [("skinny", None, 32), ("split", Path(KIND_SKINNY, 32, 16, 2, 8), 32),
            ("tiled256x128", Path(KIND_TILED, 128, 256, 1, 1), 512),
            ("wide256x256", Path(KIND_TILED, 256, 256, 1, 4), 512),
            ("tiled8wave", Path(KIND_TILED, 256, 256, 1, 8), 512),
            ("tiled128x8wave", Path(KIND_TILED, 128, 128, 1, 8), 512),
            ("tiled256x128x8wave", Path(KIND_TILED, 128, 256, 1, 8), 512)]


@pytest.mark.parametrize("fmt", [I8, FP8])
@pytest.mark.parametrize("out_dtype,out_type", [(torch.bfloat16, BF16), (torch.float16, F16)])
def test_finish_all_paths(dev, orc, fmt, out_dtype, out_type):
    N, K = 512, 1024
    rng = np.random.default_rng(fmt)
    for name, path, M in paths():
        if name in ("tiled8wave", "persistent") and fmt == FP8:
            continue
        xq, sx, wq, sw = operands(orc, M, N, K, fmt, seed=M + fmt)
        plain = gpu_gemm(dev, xq, sx, wq, sw, fmt, path=path, out_dtype=out_dtype)
        bias = (rng.standard_normal(N).astype(np.float32) * 0.5).astype(
            np.float16 if out_type == F16 else np.float32)
        bias = bias.view(np.uint16) if out_type == F16 else \
            (bias.view(np.uint32) >> 16).astype(np.uint16)
        for act in (0, 1, 2):
            for b in (bias, None):
                if act == 0 and b is None:
                    continue
                for packed in (False, True):
                    if packed and name == "split":
                        continue
                    print(f"finish {name} fmt={fmt} out={out_type} act={act} bias={b is not None} "
                          f"packed={packed}", flush=True)
                    y = run_finish(dev, xq, sx, wq, sw, fmt, b, act, path=path,
                                   out_dtype=out_dtype, packed=packed)
                    assert np.array_equal(y, orc.finish(plain, b, act, out_type))


def test_finish_grouped(dev, orc):
    """The finish also follows K-group GEMMs (decode and prefill)."""
    rng = np.random.default_rng(7)
    N, K = 256, 1024
    bias = (np.asarray(rng.standard_normal(N), np.float32).view(np.uint32) >> 16).astype(np.uint16)
    for M in (16, 512):
        xq, sx, wq, sw = operands(orc, M, N, K, I8, group=128, rotation=128, seed=M)
        plain = gpu_gemm(dev, xq, sx, wq, sw, I8, group=128)
        for act in (1, 2):
            y = run_finish(dev, xq, sx, wq, sw, I8, bias, act, group=128)
            assert np.array_equal(y, orc.finish(plain, bias, act, BF16))
