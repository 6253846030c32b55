"""The wave-specialised moment scan (sta_moments_ws: update and query waves, 64 value columns per
workgroup, queries against the state before their query block) against the oracle and against the
chunked scan (sta_moments), on both input formats and degrees 0-3, through the prefill engine.
Tolerances as elsewhere: rel-L2 1e-4 (fp32), 5e-3 (bf16 against the fp32 oracle on the upcast inputs)."""

import numpy as np
import pytest
import torch

import _engine
import _native
import reference_cpu as orc

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


def rel(a, b):
    return orc.rel_l2(torch.as_tensor(a).float().cpu(), torch.as_tensor(b).float().cpu())


CASES = [
    # n, d, dv, block, degree, semantics, dtype
    (300, 16, 16, 64, 2, "levels", torch.float32),
    (700, 64, 64, 256, 2, "levels", torch.float32),
    (513, 64, 64, 128, 2, "flat", torch.float32),
    (400, 16, 64, 128, 3, "levels", torch.float32),
    (600, 64, 64, 256, 2, "levels", torch.bfloat16),
    (257, 128, 100, 64, 2, "flat", torch.float32),
    (1000, 32, 32, 96, 1, "levels", torch.float32),
    (130, 8, 40, 64, 0, "flat", torch.float32),
    (200, 32, 32, 64, 2, "exact", torch.float32),
    (777, 64, 128, 256, 2, "levels", torch.float16),
]


@pytest.mark.parametrize("n,d,dv,block,degree,semantics,dtype", CASES)
def test_ws_moments_match_oracle_and_chunked_scan(n, d, dv, block, degree, semantics, dtype):
    print(f"ws n={n} d={d} dv={dv} block={block} degree={degree} {semantics} {dtype}", flush=True)
    q, k, v = orc.make_data((2,), n, d, dv, radius=1.0, data="unit_ball", seed=n + d)
    q, k, v = (x.to(dtype) for x in (q, k, v))
    outs = {}
    for kern in ("ws", "chunked"):
        res = _engine.prefill(q.to(DEV), k.to(DEV), v.to(DEV), degree=degree, block=block, scale=0.5,
                              semantics=semantics, compressor="none" if semantics == "exact" else "sorted_pair",
                              seed=3, moment_kernel=kern)
        outs[kern] = res.out.float().cpu()
    qf, kf, vf = (x.float() for x in (q, k, v))
    tol = 1e-4 if dtype == torch.float32 else 5e-3
    for h in range(2):
        if semantics == "levels":
            ref = orc.levels_forward(qf[h], kf[h], vf[h], degree=degree, block=block, scale=0.5, seed=3 + h)
        elif semantics == "flat":
            ref = orc.fast_path_forward(qf[h], kf[h], vf[h], degree=degree, block=block, scale=0.5, seed=3 + h)
        else:
            ref = orc.classical_attention(qf[h], kf[h], vf[h], 0.5)
        assert rel(outs["ws"][h], ref) < tol
        assert rel(outs["chunked"][h], ref) < tol
    # the two scans sum the same products in different orders: a few fp32 ulps of the sums apart
    assert rel(outs["ws"], outs["chunked"]) < (1e-5 if dtype == torch.float32 else 2e-3)


def test_ws_raw_moments_against_closed_form():
    """The query-block moments themselves: with the residual over the whole block (flat semantics at a
    block longer than the sequence the moments are everything before the row's block, i.e. nothing),
    run the scan at query blocks of 64 via exact semantics and compare low_num / low_den partials with
    the closed-form sums over the keys before each row's block."""
    n, d, dv, qb = 300, 16, 24, 64
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, n, d, generator=g) * 0.4
    k = torch.randn(1, n, d, generator=g) * 0.4
    v = torch.randn(1, n, dv, generator=g)
    lib = _native.lib()
    import _plan
    ft = _plan.feature_tiles(d, 2)
    ct = 4 if (-(-dv // 32)) % 2 == 0 else 2
    ms = _plan.moment_split_ws(ft, 1, dv, _native.moment_ws_slot_tiles(d, 2, ct, dv), ct)
    quads = torch.from_numpy(ms.quads.view(np.int32)).to(DEV)
    coef = torch.from_numpy(_plan.tile_coefficients(ms.quads, ms.coef, d)).to(DEV)
    ldv = 32 * -(-dv // 32)
    vp = torch.zeros(1, n, ldv)
    vp[..., :dv] = v
    hand = torch.empty(lib.sta_moments_ws_handoff_bytes(1, ms.fsplit, ms.wave_tiles, ct, dv) // 4, device=DEV)
    rows, ld, off = _native.moment_partials_layout(n, dv)
    low_num = torch.zeros(1, ms.fsplit, rows, ld, device=DEV)
    low_den = torch.zeros(1, ms.fsplit, rows, device=DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), vp.to(DEV)
    st = lib.sta_moments_ws(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), 0, 1, n, d, dv, ldv, 2, 0.5, qb, 0, ms.fsplit,
                            ms.wave_tiles, int(ms.mixed), ct, quads.data_ptr(), coef.data_ptr(), hand.data_ptr(),
                            low_num.data_ptr(), low_den.data_ptr(), _native.stream_handle(DEV))
    _native.check(st, "sta_moments_ws")
    num = low_num.sum(1)[0, off:off + n, :dv].cpu().double()
    den = low_den.sum(1)[0, off:off + n].cpu().double()
    x = (q[0].double() @ k[0].double().T) * 0.5
    p = orc.exp_taylor(x, 2)
    i = torch.arange(n)
    before = (i[None, :] < (i[:, None] // qb * qb))
    p = torch.where(before, p, torch.zeros_like(p))
    assert rel(num, p @ v[0].double()) < 2e-5
    assert rel(den, p.sum(-1)) < 2e-5


def test_ws_rejects_bad_arguments():
    """Refusals before any launch; every pointer is a real device buffer sized for the arguments, so a
    validation slip would give a wrong status, not a stray access."""
    lib = _native.lib()
    bh, n, d, dv, fsplit, nts = 1, 64, 64, 64, 8, 5
    q = torch.zeros((bh, n, d), device=DEV)
    k = torch.zeros((bh, n, d), device=DEV)
    v = torch.zeros((bh, n, dv), device=DEV)
    quads = torch.zeros(fsplit * 4 * nts * 4, device=DEV, dtype=torch.int32)
    coef = torch.zeros(fsplit * 4 * nts * 16, device=DEV)
    hand = torch.zeros(max(lib.sta_moments_ws_handoff_bytes(bh, fsplit, nts, 4, dv), 16) // 4, device=DEV)
    rows, ld, _ = _native.moment_partials_layout(n, dv)
    low_num = torch.zeros((bh, fsplit, rows, ld), device=DEV)
    low_den = torch.zeros((bh, fsplit, rows), device=DEV)

    def call(qb=64, ct=4, dv_=dv, with_hand=True):
        return lib.sta_moments_ws(q.data_ptr(), k.data_ptr(), v.data_ptr(), 0, bh, n, d, dv_, 64, 2, 1.0, qb, 0,
                                  fsplit, nts, 1, ct, quads.data_ptr(), coef.data_ptr(),
                                  hand.data_ptr() if with_hand else None, low_num.data_ptr(), low_den.data_ptr(),
                                  None)
    # query block below two chunks or not a whole number of chunks, column tiles of 4 with an odd number
    # of 32-column groups, no handoff
    assert call(qb=32) == _native.STA_ERR_ARG
    assert call(qb=48) == _native.STA_ERR_ARG
    assert call(ct=4, dv_=32) == _native.STA_ERR_UNSUPPORTED
    assert call(with_hand=False) == _native.STA_ERR_ARG
