"""The prefill's fp16 working copies and the range they can hold.

The flash kernel multiplies fp16 operands on the MFMA units, so every q, k
and v element (after QK-RMSNorm, RoPE and, for q, the log2(e)/sqrt(D)
scale) and every cached key and value of the history is converted to fp16
on its way in. The reference computes in fp32 and has no such limit
(attentionMixer, LocalModel.hpp:2608-2659), so a finite value that fp16
cannot hold (|x| >= 65520 rounds to infinity) must not turn into a silent
inf / NaN output: the call returns 0 and names the cause, and the next call
with ordinary inputs runs as before.

bf16 brackets the limit exactly: 65280 (0x477F) is the largest bf16 value
below 65504 and converts exactly; 65536 (0x4780) is the next one up and
overflows."""
import numpy as np
import pytest

from gpu_util import say
from test_gpu_prefill import run_case
from test_gpu_mixer import run as run_mixer

pytestmark = pytest.mark.gpu

BELOW = 65280.0   # largest bf16 value fp16 holds
ABOVE = 65536.0   # smallest bf16 value that overflows fp16


def call(gpu, *, count=40, start=0, H=4, KV=2, D=128, dtype="bf16", q_big=None,
         v_big=None, cache_big=None, norm=True):
    """one prefill of ordinary N(0, 1) inputs with one planted element"""
    import torch
    torch_type = torch.bfloat16 if dtype == "bf16" else torch.float32
    g = torch.Generator(device="cpu").manual_seed(5)

    def normal(*shape):
        return torch.randn(*shape, generator=g).to(torch_type).cuda()

    q, k, v = normal(count, H, D), normal(count, KV, D), normal(count, KV, D)
    cap = start + count
    kc = torch.zeros((KV, cap, D), dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros((KV, cap, D), dtype=torch.bfloat16, device="cuda")
    kc[:, :start] = normal(KV, start, D).to(torch.bfloat16)
    vc[:, :start] = normal(KV, start, D).to(torch.bfloat16)
    if q_big is not None:
        q[count // 2, 1, 7] = q_big
    if v_big is not None:
        v[count - 1, 1, 3] = v_big
    if cache_big is not None:
        vc[0, start // 2, 5] = cache_big
    gn = torch.ones(D, dtype=torch.float32, device="cuda") if norm else None
    out = torch.zeros((count, H, D), dtype=torch.float32, device="cuda")
    say("prefill fp16 range", dict(count=count, start=start, D=D, dtype=dtype, q_big=q_big, v_big=v_big,
                                   cache_big=cache_big, norm=norm))
    gpu.prefill(q, k, v, out, kc, vc, start, H, KV, D, q_norm=gn, k_norm=gn)
    torch.cuda.synchronize()
    return out


def expect_range_error(gpu, **kw):
    with pytest.raises(gpu.AiGpuError, match="fp16"):
        call(gpu, **kw)
    assert "65504" in gpu.last_error()


@pytest.mark.parametrize("D,dtype", [(128, "bf16"), (64, "bf16"), (64, "f32")])
def test_new_value_beyond_fp16_fails(gpu, D, dtype):
    expect_range_error(gpu, D=D, dtype=dtype, v_big=ABOVE)


@pytest.mark.parametrize("D", [128, 64])
def test_cached_value_beyond_fp16_fails(gpu, D):
    expect_range_error(gpu, D=D, start=37, cache_big=ABOVE)


def test_query_beyond_fp16_after_scale_fails(gpu):
    """without QK-RMSNorm the raw q reaches the conversion: 1e6 * log2(e) / sqrt(128)
    is 1.3e5"""
    expect_range_error(gpu, norm=False, q_big=1e6)


def test_values_at_the_limit_pass(gpu):
    out = call(gpu, start=37, v_big=BELOW, cache_big=-BELOW).cpu().numpy()
    assert np.isfinite(out).all()
    # a normed q row absorbs a large element: no overflow, no error
    out = call(gpu, q_big=1e6).cpu().numpy()
    assert np.isfinite(out).all()


def test_an_ordinary_call_after_the_error_matches_the_oracle(gpu):
    expect_range_error(gpu, v_big=ABOVE)
    ref, got, *_ = run_case(gpu, 70, 19, 8, 2, 128, 11)
    from common import assert_bf16_parity
    assert_bf16_parity(ref, got, "after a range error")


def test_mixer_value_projection_beyond_fp16_fails(gpu):
    """hidden states scaled by 1e5 project to values of ~N(0, 1e10) (weights
    ~ N(0, 1/hidden)): the v GEMM's epilogue converts them into the fp16 copy"""
    with pytest.raises(RuntimeError, match="fp16"):
        run_mixer(gpu, x_scale=1e5)
    run_mixer(gpu)   # and the next call is unaffected
