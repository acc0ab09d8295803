"""The prefill's fp16 working copies and the range they can hold.

The flash kernel multiplies fp16 operands on the MFMA units, so every q, k
and v element (after QK-RMSNorm, RoPE and, for q, the log2(e)/sqrt(D)
scale) and every cached key and value of the history is converted to fp16
on its way in. The reference computes in fp32 and has no such limit
(attentionMixer, LocalModel.hpp:2608-2659), so a finite value that fp16
cannot hold (|x| >= 65520 rounds to infinity) must not turn into a silent
inf / NaN output. The device-form calls are asynchronous: each takes a
ticket, its kernels raise the ticket's flag, and aigpu_range_status
(check_range here) names the earliest offending call. The host form waits
for its kernels and fails itself.

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


def inputs(*, count=40, start=0, H=4, KV=2, D=128, dtype="bf16", q_big=None, v_big=None, cache_big=None,
           norm=True):
    """ordinary N(0, 1) inputs with one planted element"""
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
    return dict(q=q, k=k, v=v, kc=kc, vc=vc, gn=gn, out=out, start=start, H=H, KV=KV, D=D)


def launch(gpu, x, check=True):
    """one device-form prefill; returns its ticket"""
    gpu.prefill(x["q"], x["k"], x["v"], x["out"], x["kc"], x["vc"], x["start"], x["H"], x["KV"], x["D"],
                q_norm=x["gn"], k_norm=x["gn"], check=check)
    return gpu.range_ticket()


def call(gpu, **kw):
    x = inputs(**kw)
    launch(gpu, x)
    return x["out"]


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


def test_asynchronous_calls_report_the_offending_ticket(gpu):
    """the device form returns without waiting; a later status query names the
    ticket of the call that overflowed, not of the ordinary calls around it,
    and leaves every flag clear"""
    gpu.check_range()   # start clear
    good = inputs(count=33)
    bad = inputs(count=40, v_big=ABOVE)
    before = launch(gpu, good, check=False)
    offending = launch(gpu, bad, check=False)
    after = launch(gpu, good, check=False)
    assert before + 1 == offending and offending + 1 == after
    with pytest.raises(gpu.AiGpuError, match="fp16") as err:
        gpu.check_range()
    assert err.value.ticket == offending
    assert f"ticket {offending}" in str(err.value)
    gpu.check_range()   # the flags are clear again


def test_host_form_fails_its_own_call(gpu):
    """aigpu_prefill_attention_host waits for its kernels and fails itself;
    the next host call with ordinary inputs runs and matches the device form"""
    x = inputs(count=40, v_big=ABOVE, dtype="f32")
    args = (x["kc"], x["vc"], 0, x["H"], x["KV"], x["D"])
    gn = x["gn"].cpu().numpy()
    with pytest.raises(gpu.AiGpuError, match="fp16"):
        gpu.prefill_host(x["q"].cpu().numpy(), x["k"].cpu().numpy(), x["v"].cpu().numpy(), *args,
                         q_norm=gn, k_norm=gn)
    gpu.check_range()   # the host form cleared its own flag
    y = inputs(count=40, dtype="f32")
    got = gpu.prefill_host(y["q"].cpu().numpy(), y["k"].cpu().numpy(), y["v"].cpu().numpy(), y["kc"], y["vc"], 0,
                           y["H"], y["KV"], y["D"], q_norm=gn, k_norm=gn)
    launch(gpu, y)
    np.testing.assert_array_equal(got, y["out"].cpu().numpy())


def test_mixer_value_projection_beyond_fp16_fails(gpu):
    """hidden states scaled by 1e5 project to values of ~N(0, 1e10) (weights
    ~ N(0, 1/hidden)): the v GEMM's epilogue converts them into the fp16 copy"""
    with pytest.raises(RuntimeError, match="fp16"):
        run_mixer(gpu, x_scale=1e5)
    run_mixer(gpu)   # and the next call is unaffected


def test_fused_kv_projection_beyond_fp16_fails(gpu):
    """at a shape where k and v run as one DMA GEMM followed by
    kv_epilogue_kernel (8192 rows, 2 KV D = 2048 columns), the epilogue's
    conversion raises the flag; an ordinary call afterwards matches the oracle"""
    kw = dict(count=8192, start=40, hidden=64, H=16, KV=8, D=128, window=64)
    with pytest.raises(RuntimeError, match="fp16"):
        run_mixer(gpu, "bf16", x_scale=1e5, **kw)
    run_mixer(gpu, "bf16", **kw)
