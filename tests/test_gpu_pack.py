"""HIP packers vs the CPU oracle: bit-exact uint32 (pack_q / unpack_q) and
nibble (pack_nibbles / unpack_nibbles) layouts, the reference's known answer,
aligned (vector) and misaligned (scalar) buffers, numpy round trips."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import packing_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_pack_known_answer_on_gpu():
    from mlx_gptq import packing

    words = packing.pack_mxfp4(np.arange(16, dtype=np.uint8))
    assert words.dtype == np.uint32 and words.tolist() == [0x76543210, 0xFEDCBA98]
    assert packing.unpack_q(words, 4, 16).tolist() == list(range(16))


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("shape", [(1, 64), (7, 96), (3, 5, 2048), (257, 4096)])
def test_pack_q_bit_exact(bits, shape):
    from mlx_gptq import packing

    rng = np.random.default_rng(bits + shape[-1])
    q = rng.integers(0, 256, shape).astype(np.uint8)  # unmasked codes, as numpy allows
    ref = packing_ref.pack_q(q, bits)
    got = packing.pack_q(torch.from_numpy(q).to(DEV), bits)
    assert got.shape == ref.shape
    np.testing.assert_array_equal(got.cpu().view(torch.int32).numpy().view(np.uint32), ref)
    np.testing.assert_array_equal(packing.pack_q(q, bits), ref)
    back = packing.unpack_q(ref, bits, shape[-1])
    np.testing.assert_array_equal(back, packing_ref.unpack_q(ref, bits, shape[-1]))


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_pack_q_misaligned_views(bits):
    from mlx_gptq import packing

    per = 32 // bits
    rng = np.random.default_rng(11)
    base = torch.from_numpy(rng.integers(0, 2**bits, 1 + 37 * per * 9).astype(np.uint8)).to(DEV)
    q = base[1:].reshape(37, per * 9)  # 1-byte offset: scalar path
    got = packing.pack_q(q, bits).cpu().view(torch.int32).numpy().view(np.uint32)
    np.testing.assert_array_equal(got, packing_ref.pack_q(q.cpu().numpy(), bits))


@pytest.mark.parametrize("shape", [(5, 64), (3, 7, 2048), (1, 2), (129, 34)])
def test_nibbles_bit_exact(shape):
    from mlx_gptq import artifacts

    q = torch.randint(0, 256, shape, dtype=torch.uint8)
    ref = packing_ref.pack_nibbles(q)
    got = artifacts.pack_nibbles(q.to(DEV))
    assert torch.equal(got.cpu(), ref)
    assert torch.equal(artifacts.unpack_nibbles(got).cpu(), packing_ref.unpack_nibbles(ref))
    q16 = q & 0xF
    assert torch.equal(artifacts.unpack_nibbles(artifacts.pack_nibbles(q16.to(DEV))).cpu(), q16)


def test_nibble_and_word_layouts_agree_on_gpu():
    from mlx_gptq import artifacts, packing

    q = torch.randint(0, 16, (5, 64), dtype=torch.uint8, device=DEV)
    w = packing.pack_q(q, 4)
    assert torch.equal(w.view(torch.uint8).reshape(5, 32), artifacts.pack_nibbles(q))
