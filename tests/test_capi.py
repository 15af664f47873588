"""The C-ABI library without a GPU: it loads, exports every symbol include/foidfinder_rocm.h declares, and rejects
bad arguments with FF_EINVAL and a message before any HIP call (the reference raises RuntimeError via TORCH_CHECK
for the same preconditions, foidfinder/backends/cuda/csrc/kernels.cu:190-205, :222, :240, :257-258)."""

from __future__ import annotations

import re
from pathlib import Path

import pytest
import torch

from foidfinder_amd import kernels as K

HEADER = Path(__file__).resolve().parents[1] / "include" / "foidfinder_rocm.h"
FF_OK, FF_EINVAL = 0, 1


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"\b(ff_\w+)\s*\(", text)


def test_library_exports_every_declared_symbol():
    names = declared()
    assert {"ff_rot_q8_1024", "ff_rot_q8_h128", "ff_gemm_s8", "ff_attention", "ff_last_error"} <= set(names)
    lib = K.lib()
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(K.SIGNATURES), "ctypes signatures must cover the header exactly"


def test_abi_version_and_variants():
    lib = K.lib()
    assert lib.ff_abi_version() == K.ABI_VERSION
    assert lib.ff_gemm_s8_variants() >= 1


def err(status):
    return status, K.lib().ff_last_error().decode()


def test_rot_q8_1024_rejects_bad_arguments():
    lib = K.lib()
    assert err(lib.ff_rot_q8_1024(None, None, None, 1e-5, -1, None, None, None)) == (FF_EINVAL, "rot_q8_1024: T must be >= 0")
    assert lib.ff_rot_q8_1024(None, None, None, 1e-5, 0, None, None, None) == FF_OK  # empty input: nothing to do
    assert err(lib.ff_rot_q8_1024(None, None, None, 1e-5, 4, None, None, None))[0] == FF_EINVAL
    s, m = err(lib.ff_rot_q8_1024(16, 16, None, 1e-5, 4, 16, 16, None))
    assert s == FF_EINVAL and "gamma and beta" in m
    s, m = err(lib.ff_rot_q8_1024(16, 16, 16, 0.0, 4, 16, 16, None))
    assert s == FF_EINVAL and "eps" in m
    s, m = err(lib.ff_rot_q8_1024(18, None, None, 1e-5, 4, 16, 16, None))
    assert s == FF_EINVAL and "misaligned" in m


def test_rot_q8_h128_rejects_bad_arguments():
    lib = K.lib()
    for C in (0, 100, 6272):
        s, m = err(lib.ff_rot_q8_h128(16, 4, C, 0, None, None, 0.0, 16, 16, None))
        assert s == FF_EINVAL and "C" in m
    s, m = err(lib.ff_rot_q8_h128(16, 4, 256, 300, 16, 16, 1e-6, 16, 16, None))
    assert s == FF_EINVAL and "c_real" in m


def test_gemm_s8_rejects_bad_arguments():
    lib = K.lib()

    def call(M=8, N=16, Kd=64, epi=4, variant=0, rope=(None, None, 0), ptrs=256):
        return err(lib.ff_gemm_s8(ptrs, ptrs, M, N, Kd, ptrs, ptrs, ptrs, ptrs, epi, variant, rope[0], rope[1], rope[2],
                                  1.0, None))

    assert call(Kd=100)[1] == "gemm_s8: K must be a multiple of 64"
    assert call(N=40)[1] == "gemm_s8: N must be a multiple of 16"
    assert "epilogue" in call(epi=9)[1]
    assert "variant" in call(variant=99)[1]
    assert "QKV" in call(N=48, epi=0)[1]  # N = 3C needs C % 64 == 0
    assert "RoPE" in call(N=192, epi=0)[1]
    assert "rope_len" in call(N=192, epi=0, rope=(256, 256, 1 << 24))[1]  # table bytes must fit 31 bits
    assert "rope_len" not in call(N=192, epi=0, rope=(256, 256, (1 << 24) - 1), ptrs=8)[1]  # largest accepted
    assert call(M=0) == (FF_OK, "")
    assert "misaligned" in call(ptrs=8)[1]
    assert "not supported" in call(Kd=(1 << 22) + 64)[1]  # 32-bit offsets within a tile
    assert "not supported" in call(N=(1 << 21) + 16)[1]


def test_attention_rejects_bad_arguments():
    lib = K.lib()
    assert "multiple of seq_len" in err(lib.ff_attention(16, 16, 10, 16, 3, None))[1]
    assert "heads" in err(lib.ff_attention(16, 16, 10, 0, 5, None))[1]
    assert "seq_len" in err(lib.ff_attention(16, 16, 10, 16, 0, None))[1]
    assert lib.ff_attention(None, None, 0, 16, 5, None) == FF_OK


def test_python_ops_refuse_cpu_tensors():
    x = torch.zeros(4, 1024, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="GPU tensors"):
        K.rot_q8_1024(x, None, None, torch.zeros(4, 1024, dtype=torch.int8), torch.zeros(4), 1e-5)
    with pytest.raises((RuntimeError, NotImplementedError)):  # no CPU kernel is registered for the op
        torch.ops.foidfinder_rocm.attention(torch.zeros(5, 192, dtype=torch.float16), torch.zeros(5, 64, dtype=torch.float16), 5)


def test_op_schemas_mirror_the_reference():
    ops = K.kernels()
    schema = str(ops.gemm_s8.default._schema)
    assert "Tensor(a!) out, int epi, int stages, Tensor? rope_cos, Tensor? rope_sin, float q_scale" in schema
    assert "Tensor(a!) out, Tensor(b!) row_scale" in str(ops.rot_q8_1024.default._schema)
    assert "attention(Tensor qkv, Tensor(a!) out, int seq_len)" in str(ops.attention.default._schema)


def test_resample_u8_rejects_bad_arguments():
    lib = K.lib()

    def call(src=(100, 80), axis=0, ksize=5, row0=0, out=(448, 448), region=(0, 0, 100, 40), ptrs=256):
        top, left, h, w = region
        return err(lib.ff_resample_u8(ptrs, src[0], src[1], axis, ptrs, ptrs, ksize, row0, ptrs, out[0], out[1], top,
                                      left, h, w, None))

    assert "axis" in call(axis=2)[1]
    assert "positive" in call(ksize=0)[1]
    assert "positive" in call(region=(0, 0, 0, 40))[1]
    assert "inside the output" in call(region=(400, 0, 100, 40))[1]
    assert "inside the output" in call(region=(0, -1, 10, 40))[1]
    assert "outside the source" in call(row0=1)[1]  # axis 0 reads rows row0 .. row0 + h - 1 of 100
    assert "outside the source" in call(axis=1, region=(0, 0, 10, 81))[1]  # axis 1 reads columns 0 .. w - 1 of 80
    assert "65535" in call(src=(70000, 3))[1]
    assert "null" in call(ptrs=None)[1]


def test_pool_kernels_reject_bad_arguments():
    lib = K.lib()
    assert "C <= 2048" in err(lib.ff_layer_norm2(256, 4, 100, 256, 256, 256, 256, 1e-6, 256, None))[1]
    assert "eps" in err(lib.ff_layer_norm2(256, 4, 768, 256, 256, 256, 256, 0.0, 256, None))[1]
    assert lib.ff_layer_norm2(None, 0, 768, None, None, None, None, 1e-6, None, None) == FF_OK
    assert lib.ff_slot_weights_blocks(1025) == 33 and lib.ff_slot_weights_blocks(0) == 0

    def sw(B=2, N=1025, G=16, M=18, c_stride=0, ptrs=256):
        return err(lib.ff_slot_weights(ptrs, ptrs, c_stride, ptrs, B, N, G, M, ptrs, ptrs, None))

    assert "M must be 6 or 18" in sw(M=7)[1]
    assert "bad B, N or G" in sw(N=0)[1]
    assert "c_stride" in sw(c_stride=5)[1]
    assert "LDS" in sw(G=64)[1]
    assert "null" in sw(ptrs=None)[1]
    assert sw(B=0) == (FF_OK, "")
