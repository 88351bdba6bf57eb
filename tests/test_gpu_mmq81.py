"""GPU parity of hip_gemm_q8_1_mmq (ggml-cuda's int8 MMQ rounding for Q4_K /
Q6_K) against the oracle's restatement of gemm_q4k_q8_1_mmq /
gemm_q6k_q8_1_mmq[_stream_k] (src/dequant.rs:202-645): bit-exact, including
the stream-K split (tail + prefix)."""
import numpy as np
import pytest

from saient_quartz_amd import synth
from saient_quartz_amd.api import check
from saient_quartz_amd.host import GpuBuf

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("t", [12, 14])
@pytest.mark.parametrize("rows, in_dim, out_dim", [(1, 256, 37), (3, 1024, 300), (16, 4096, 64), (17, 512, 129),
                                                   (40, 2048, 16)])
@pytest.mark.parametrize("stream_k", [None, (128, 2), (300, 7)])
def test_gemm_q8_1_mmq_bit_exact(qh, oracle, t, rows, in_dim, out_dim, stream_k):
    rng = np.random.default_rng(rows * 7 + in_dim + out_dim + t)
    x = (rng.standard_normal((rows, in_dim)) * rng.uniform(0.01, 30)).astype(np.float32)
    x[0, :32] = 0.0  # an all-zero Q8_1 block
    data = synth.weights(t, out_dim, in_dim, seed=rows + out_dim)
    ref_rows, mps = stream_k if stream_k else (0, 0)
    want = oracle.gemm_q8_1_mmq(t, x, data, in_dim, out_dim, rows, ref_rows, mps)
    dw, dx, dy = GpuBuf.upload(data), GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.alloc_f32(rows * out_dim)
    check("hip_gemm_q8_1_mmq", qh.hip_gemm_q8_1_mmq(t, dw.ptr, dx.ptr, dy.ptr, in_dim, out_dim, rows, ref_rows, mps))
    check("hip_sync", qh.hip_sync())
    got = dy.download(np.float32)[:rows * out_dim].reshape(rows, out_dim)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), np.argwhere(got != want)[:5]


def test_gemm_q8_1_mmq_stream_k_changes_bits(qh, oracle):
    """The stream-K cut is exercised: some outputs differ in their last bits from
    the unsplit accumulation, and the GPU follows the split one."""
    rows, in_dim, out_dim = 2, 1024, 384
    x = np.random.default_rng(9).standard_normal((rows, in_dim)).astype(np.float32)
    data = synth.weights(12, out_dim, in_dim, seed=9)
    plain = oracle.gemm_q8_1_mmq(12, x, data, in_dim, out_dim, rows)
    split = oracle.gemm_q8_1_mmq(12, x, data, in_dim, out_dim, rows, 128, 2)
    assert not np.array_equal(plain, split)
    dw, dx, dy = GpuBuf.upload(data), GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.alloc_f32(rows * out_dim)
    check("mmq", qh.hip_gemm_q8_1_mmq(12, dw.ptr, dx.ptr, dy.ptr, in_dim, out_dim, rows, 128, 2))
    check("hip_sync", qh.hip_sync())
    assert np.array_equal(dy.download(np.float32)[:rows * out_dim].reshape(rows, out_dim), split)
