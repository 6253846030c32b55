"""sta_decode_step_static, the decode step that allocates nothing (its moment partials live in the
library's static device scratch), through the C ABI on the GPU: its outputs equal the allocating path
(sta_decode_moments + sta_decode_tail on caller buffers) bit for bit, token after token, on two calls in
a row of which the second is smaller, and without a moment state (compressor "none", zeroed partials)."""

import pytest
import torch

import _native
import streaming_taylor_coreset_attention as stc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def _lockstep(streams, d, dv, block, prefix, steps, compressor="sorted_pair", dtype=torch.float32, seed=0):
    """Two identical states: one advanced with step(), the other with step_into() wherever the token
    does not complete a block; every output compared bit for bit."""
    print(f"no-alloc lockstep: S={streams} d={d} dv={dv} block={block} prefix={prefix} steps={steps} "
          f"{compressor} {dtype}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(1000 + streams)
    n = prefix + steps
    q, k, v = ((torch.randn(streams, n, w, generator=g, device=DEV) * 0.125).to(dtype) for w in (d, d, dv))
    ref, st = (stc.ArticleStreamingAttention(d, dv, degree=2, block_size=block, scale=0.125, compressor=compressor,
                                             device=DEV, dtype=dtype, seed=seed, streams=streams) for _ in range(2))
    if prefix:
        ref.extend(k[:, :prefix], v[:, :prefix])
        st.extend(k[:, :prefix], v[:, :prefix])
    out = torch.empty((streams, dv), device=DEV, dtype=dtype)
    used = 0
    for i in range(prefix, n):
        qi, ki, vi = q[:, i].contiguous(), k[:, i].contiguous(), v[:, i].contiguous()
        want = ref.step(qi, ki, vi)
        s = st._st
        if (not s.exact and s.buf_len + 1 == s.block) or (s.exact and s.buf_len == s.cap):
            got = st.step(qi, ki, vi)
        else:
            got = st.step_into(qi, ki, vi, out).clone()
            used += 1
        assert torch.equal(got, want), f"token {i}"
    torch.cuda.synchronize()
    st.release_static()
    assert used >= steps - steps // block - 1
    return used


def test_static_step_matches_allocating_step_then_a_smaller_call():
    # first call: 512 streams, d = dv = 64, through a block completion and the level merges around it
    _lockstep(512, 64, 64, 64, prefix=200, steps=70)
    # second call, smaller (fewer streams, narrower rows): the scratch keeps the first call's contents,
    # every partial it reads must have been rewritten
    _lockstep(24, 32, 40, 32, prefix=45, steps=40)


def test_static_step_bf16_and_without_moment_state():
    _lockstep(64, 64, 64, 64, prefix=100, steps=40, dtype=torch.bfloat16)
    _lockstep(16, 16, 48, 32, prefix=10, steps=30, compressor="none")


def test_static_step_refuses_a_working_set_beyond_the_scratch():
    """A working set beyond the static scratch is refused before any launch.  Every pointer is a real
    device buffer sized for the arguments (degree 0: one feature; blocks of 2, no levels), so a
    validation slip would give a wrong status, not a stray access."""
    lib = _native.lib()
    cap = lib.sta_static_scratch_bytes()
    assert cap == 16 << 20
    d, dv, splits, block = 64, 64, 1, 2
    streams = cap // (4 * (dv + 1)) + 64  # partials of this many streams exceed the scratch
    z = dict(device=DEV, dtype=torch.float32)
    q, k, v = torch.zeros((streams, d), **z), torch.zeros((streams, d), **z), torch.zeros((streams, dv), **z)
    state_num, state_den = torch.zeros((streams, 1, dv), **z), torch.zeros((streams, 1), **z)
    findex = torch.zeros(1, device=DEV, dtype=torch.int32)
    buf_k, buf_v = torch.zeros((streams, block, d), **z), torch.zeros((streams, block, dv), **z)
    lev = torch.zeros(4, **z)
    out = torch.zeros((streams, dv), **z)
    st = lib.sta_decode_step_static(q.data_ptr(), k.data_ptr(), v.data_ptr(), 0, streams, d, dv, 0, 0.125, 1e-12,
                                    _native.DEC_QUERY, state_num.data_ptr(), state_den.data_ptr(), 1,
                                    findex.data_ptr(), 4, splits, buf_k.data_ptr(), buf_v.data_ptr(), block, 0,
                                    lev.data_ptr(), lev.data_ptr(), lev.data_ptr(), 0, 1, 0, out.data_ptr(), 0, None,
                                    None)
    assert st == _native.STA_ERR_SCRATCH
    assert b"static scratch" in lib.sta_status_string(st)


def test_static_scratch_serves_one_object_and_stream_at_a_time():
    """The device's static scratch is claimed by the first object's step_into on its stream; another
    object's step_into, or the same object's on another stream, is refused (their partials would
    overwrite each other) until release_static()."""
    print("no-alloc owner check", flush=True)
    d, dv, s_ = 16, 16, 4
    a, b = (stc.ArticleStreamingAttention(d, dv, degree=2, block_size=64, scale=0.25, device=DEV, streams=s_)
            for _ in range(2))
    x = torch.randn(s_, d, device=DEV) * 0.25
    y = torch.randn(s_, dv, device=DEV)
    out = torch.empty(s_, dv, device=DEV)
    a.step_into(x, x, y, out)
    with pytest.raises(ValueError, match="another decode state"):
        b.step_into(x, x, y, out)
    side = torch.cuda.Stream(device=DEV)
    with torch.cuda.stream(side):
        with pytest.raises(ValueError, match="another stream"):
            a.step_into(x, x, y, out)
    a.release_static()
    b.step_into(x, x, y, out)
    want = a.step(x, x, y)  # a's second token, allocating path
    got = b.step_into(x, x, y, out)  # b's second token: the same inputs, so the same outputs
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    b.release_static()
