"""Launch timing through ``lik_launch_opts_t::timing_start / timing_stop``
(``_lib.LaunchTimer`` with ``launch_options(timer=...)``, what bench.py's
roofline uses). The library passes the events to the scoring launches
themselves (hipExtLaunchKernel), so:

* a timed call returns bitwise the scores of an untimed one;
* every timed call yields one event pair with a positive duration, no longer
  than the wall time of the calls, including a doc mask with holes (two
  scoring launches: the span runs from the first one's start to the last
  one's end), the KD layout (the streaming kernel of lik_q1.hip) and packed
  docs;
* the events are host-created (hipEventCreate): the timer queues nothing on
  the stream.
"""

import sys

import pytest
import torch

from late_interaction_kernels._lib import LaunchTimer, launch_options

pytestmark = pytest.mark.gpu


def _case(tag):
    print(f"[case] {tag}", flush=True)
    sys.stdout.flush()


def _timed(fn, n=4):
    timer = LaunchTimer()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with launch_options(timer=timer):
        start.record()
        outs = [fn() for _ in range(n)]
        end.record()
    torch.cuda.synchronize()
    kms, launches = timer.total_ms()
    return outs, kms, launches, start.elapsed_time(end)


def _check(fn, n=4):
    ref = fn()
    outs, kms, launches, wall = _timed(fn, n)
    assert launches == n
    assert 0.0 < kms <= wall * 1.01 + 0.05
    for o in outs:
        assert torch.equal(o, ref)
    return kms / n


def test_timing_dense_mask_with_holes():
    from late_interaction_kernels import maxsim

    _case("timing dense, mask with holes")
    g = torch.Generator(device="cuda").manual_seed(3)
    Q = torch.randn(64, 32, 128, generator=g, device="cuda").to(torch.bfloat16)
    D = torch.randn(512, 200, 128, generator=g, device="cuda").to(torch.bfloat16)
    lens = torch.randint(20, 201, (512,), generator=g, device="cuda")
    dm = torch.arange(200, device="cuda")[None] < lens[:, None]
    dm[::7, 5] = False  # holes: those docs take the second (masked) launch
    _check(lambda: maxsim(Q, D, d_mask=dm, normalize=False))


def test_timing_kd_stream_kernel():
    from late_interaction_kernels import maxsim

    _case("timing KD layout")
    g = torch.Generator(device="cuda").manual_seed(4)
    Q = torch.randn(32, 32, 128, generator=g, device="cuda").to(torch.bfloat16)
    D = torch.randn(32, 16, 150, 128, generator=g, device="cuda").to(torch.bfloat16)
    lens = torch.randint(1, 151, (32, 16), generator=g, device="cuda")
    dm = torch.arange(150, device="cuda")[None, None] < lens[..., None]
    _check(lambda: maxsim(Q, D, d_mask=dm, normalize=False))


def test_timing_varlen():
    from late_interaction_kernels import maxsim_varlen

    _case("timing varlen")
    g = torch.Generator().manual_seed(5)
    q_lens = torch.full((16,), 32)
    d_lens = torch.randint(1, 300, (300,), generator=g)
    cu_q = torch.zeros(17, dtype=torch.int32)
    cu_q[1:] = torch.cumsum(q_lens, 0)
    cu_d = torch.zeros(301, dtype=torch.int32)
    cu_d[1:] = torch.cumsum(d_lens, 0)
    Qp = torch.randn(int(cu_q[-1]), 128, generator=g).to(torch.bfloat16).cuda()
    Dp = torch.randn(int(cu_d[-1]), 128, generator=g).to(torch.bfloat16).cuda()
    cq, cd = cu_q.cuda(), cu_d.cuda()
    _check(lambda: maxsim_varlen(Qp, Dp, cq, cd))
