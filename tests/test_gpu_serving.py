"""GPU parity of the ragged mixed prefill + decode step (kdn_ragged_step) and the state pool.

The oracle: for every sequence of the step, the float64 token recurrence (oracle.scan.token_recurrence,
or linear_recurrence for rule 1) over the oracle's structured lift (oracle.lift.lift), continuing from
the sequence's slot state; slots that no sequence uses must come back bit-identical.  Tolerances
(relative L2) as for the scan: 1e-4 for fp32 inputs, 2e-2 for bf16 inputs.  The further check the
serving path calls for: prefill followed by decode steps equals one prefill of the whole sequence.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kdn import ops
from kernels import FastWalshHadamardProjection
from oracle import lift as ol
from oracle import scan as osc
from serving import HybridMemoryPool, hybrid_recurrent_forward

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = {torch.float32: 1e-4, torch.bfloat16: 2e-2}


@pytest.fixture(scope="module")
def proj():
    return FastWalshHadamardProjection(64, 512, 42)


@pytest.fixture(scope="module")
def oproj():
    return ol.make_projection(64, 512, 42)


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def make_step(lens, H, dv, dtype, n_slots, seed, decay=True):
    g = torch.Generator().manual_seed(seed)
    T = int(sum(lens))
    q = torch.randn(T, H, 64, generator=g).to(dtype)
    k = torch.randn(T, H, 64, generator=g).to(dtype)
    v = torch.randn(T, H, dv, generator=g).to(dtype)
    beta = torch.sigmoid(torch.randn(T, H, generator=g))
    lam = (0.9 + 0.1 * torch.rand(T, H, generator=g)) if decay else None
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int64)
    slots = torch.randperm(n_slots, generator=g)[: len(lens)].to(torch.int32)
    states = 0.05 * torch.randn(n_slots, H, 512, dv, generator=g)
    return q, k, v, beta, lam, cu, slots, states


def oracle_step(q, k, v, beta, lam, cu, slots, states, oproj, normalize=False, rule=ops.RULE_DELTA):
    def rows(x):
        x = x.float()
        if normalize:  # F.normalize keeps the input dtype
            x = F.normalize(x, dim=-1, eps=1e-6).to(q.dtype).float()
        return x.numpy()

    fn = osc.token_recurrence if rule == ops.RULE_DELTA else osc.linear_recurrence
    T, H = q.shape[:2]
    Y = np.zeros((T, H, v.shape[-1]))
    S = states.double().numpy().copy()
    for i in range(len(slots)):
        lo, hi = int(cu[i]), int(cu[i + 1])
        if hi == lo:
            continue
        s = int(slots[i])
        for h in range(H):
            pq = ol.lift(rows(q[lo:hi, h]), oproj)
            pk = ol.lift(rows(k[lo:hi, h]), oproj)
            d = None if lam is None else lam[lo:hi, h].double().numpy()[None]
            y, Sf = fn(pq[None], pk[None], v[lo:hi, h].double().numpy()[None], beta[lo:hi, h].double().numpy()[None],
                       d, states[s, h].double().numpy().T[None])
            Y[lo:hi, h] = y[0]
            S[s, h] = Sf[0].T
    return Y, S


def run_step(proj, q, k, v, beta, lam, cu, slots, states, normalize=False, rule=ops.RULE_DELTA, pipelined=True):
    sd = states.to(DEV)
    y = ops.ragged_step(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), None if lam is None else lam.to(DEV), cu,
                        slots, sd, proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv,
                        normalize=normalize, rule=rule, pipelined=pipelined)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), sd.cpu()


LENS = [1, 1, 0, 37, 1, 200, 1, 64, 1, 130, 1, 1]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("decay", [False, True])
def test_mixed_step_parity(proj, oproj, dtype, decay):
    q, k, v, beta, lam, cu, slots, states = make_step(LENS, 2, 64, dtype, 20, seed=1, decay=decay)
    y, S = run_step(proj, q, k, v, beta, lam, cu, slots, states)
    Yr, Sr = oracle_step(q, k, v, beta, lam, cu, slots, states, oproj)
    assert rel_l2(y, Yr) < TOL[dtype]
    used = set(int(s) for s in slots)
    for s in range(20):
        if s in used:
            assert rel_l2(S[s].numpy(), Sr[s]) < TOL[dtype], s
        else:
            assert torch.equal(S[s], states[s]), s  # untouched slots, bit for bit


def test_decode_only_and_prefill_only(proj, oproj):
    for lens in ([1] * 9, [70, 3, 129]):
        q, k, v, beta, lam, cu, slots, states = make_step(lens, 3, 64, torch.float32, 12, seed=2)
        y, S = run_step(proj, q, k, v, beta, lam, cu, slots, states)
        Yr, Sr = oracle_step(q, k, v, beta, lam, cu, slots, states, oproj)
        assert rel_l2(y, Yr) < 1e-4
        for s in slots.tolist():
            assert rel_l2(S[s].numpy(), Sr[s]) < 1e-4


@pytest.mark.parametrize("dv", [16, 32, 128])
def test_value_widths(proj, oproj, dv):
    q, k, v, beta, lam, cu, slots, states = make_step([1, 90, 1, 1, 65], 2, dv, torch.float32, 8, seed=3)
    y, S = run_step(proj, q, k, v, beta, lam, cu, slots, states)
    Yr, Sr = oracle_step(q, k, v, beta, lam, cu, slots, states, oproj)
    assert rel_l2(y, Yr) < 1e-4
    for s in slots.tolist():
        assert rel_l2(S[s].numpy(), Sr[s]) < 1e-4


def test_normalize_and_linear_rule(proj, oproj):
    q, k, v, beta, lam, cu, slots, states = make_step([1, 77, 1, 3], 2, 64, torch.bfloat16, 6, seed=4)
    for rule in (ops.RULE_DELTA, ops.RULE_LINEAR):
        y, S = run_step(proj, q, k, v, beta, lam, cu, slots, states, normalize=True, rule=rule)
        Yr, Sr = oracle_step(q, k, v, beta, lam, cu, slots, states, oproj, normalize=True, rule=rule)
        assert rel_l2(y, Yr) < 2e-2
        for s in slots.tolist():
            assert rel_l2(S[s].numpy(), Sr[s]) < 2e-2


def test_prefill_then_decode_equals_one_prefill(proj):
    # one sequence: a prefill of 300 tokens then 5 decode steps == a prefill of 305 tokens
    g = torch.Generator().manual_seed(5)
    L, H = 305, 2
    q = torch.randn(L, H, 64, generator=g)
    k = torch.randn(L, H, 64, generator=g)
    v = torch.randn(L, H, 64, generator=g)
    beta = torch.sigmoid(torch.randn(L, H, generator=g))
    lam = 0.95 + 0.05 * torch.rand(L, H, generator=g)
    st = torch.zeros(4, H, 512, 64, device=DEV)
    slot = torch.tensor([2], dtype=torch.int32)
    ys = []
    for lo, hi in [(0, 300)] + [(t, t + 1) for t in range(300, 305)]:
        ys.append(ops.ragged_step(q[lo:hi].to(DEV), k[lo:hi].to(DEV), v[lo:hi].to(DEV), beta[lo:hi].to(DEV),
                                  lam[lo:hi].to(DEV), [0, hi - lo], slot, st, proj.device_omega(DEV),
                                  proj.device_phase(DEV), proj.tau_star_inv))
    y_steps = torch.cat(ys, 0)
    st1 = torch.zeros(4, H, 512, 64, device=DEV)
    y_one = ops.ragged_step(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), [0, L], slot, st1,
                            proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv)
    torch.cuda.synchronize()
    assert rel_l2(y_steps.cpu().numpy(), y_one.cpu().numpy()) < 1e-5
    assert rel_l2(st.cpu().numpy(), st1.cpu().numpy()) < 1e-5


def test_serving_op_with_reference_state_layout(proj, oproj):
    # recurrent_states [slots, H, d_v, D] and a token -> slot mapping, as the reference op takes them
    lens = [1, 40, 1, 1, 25]
    q, k, v, beta, lam, cu, slots, states = make_step(lens, 2, 64, torch.float32, 7, seed=6)
    slot_mapping = torch.repeat_interleave(slots.to(torch.int64), torch.tensor(lens))
    rs = states.transpose(2, 3).contiguous().to(DEV)   # [slots, H, d_v, D]
    out = torch.empty(q.shape[0], 2, 64, device=DEV)
    hybrid_recurrent_forward(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), rs, slot_mapping.to(DEV),
                             out, fwht_proj=proj)
    torch.cuda.synchronize()
    Yr, Sr = oracle_step(q, k, v, beta, lam, cu, slots, states, oproj)
    assert rel_l2(out.cpu().numpy(), Yr) < 1e-4
    for s in slots.tolist():
        assert rel_l2(rs[s].transpose(1, 2).cpu().numpy(), Sr[s]) < 1e-4


def test_pool_zeroes_and_forks_on_device(proj):
    pool = HybridMemoryPool(6, 1024, num_layers=2, num_heads=2, device=DEV)
    pool.slab.fill_(3.0)
    a = pool.allocate_stream(10)
    assert float(pool.slab[a].abs().max()) == 0.0          # a new stream starts from S = 0
    pool.slab[a].normal_()
    b = pool.fork_stream(a)
    torch.cuda.synchronize()
    assert torch.equal(pool.slab[b], pool.slab[a])
    assert float(pool.slab[b + 1].min()) == 3.0             # other slots untouched
    # a step on layer 1 through the pool's layer view updates only the used slot of that layer
    before = pool.slab.clone()
    q, k, v, beta, lam, cu, slots, _ = make_step([1], 2, 64, torch.float32, 1, seed=7)
    ops.ragged_step(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), cu, torch.tensor([b], dtype=torch.int32),
                    pool.layer_states(1), proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv)
    torch.cuda.synchronize()
    changed = (pool.slab != before).reshape(6, 2, -1).any(-1)
    assert changed[b, 1] and int(changed.sum()) == 1


def test_caller_workspace_reused_across_steps(proj):
    # a serving loop sizes one workspace with ragged_workspace_bytes and passes it to every step: the same
    # results, bit for bit, as steps that allocate their own
    q, k, v, beta, lam, cu, slots, states = make_step(LENS, 2, 64, torch.bfloat16, 20, seed=5, decay=True)
    dq, dk, dv, db, dl = (t.to(DEV) for t in (q, k, v, beta, lam))
    om, ph = proj.device_omega(DEV), proj.device_phase(DEV)
    need = ops.ragged_workspace_bytes(dq, dk, dv, db, dl, cu, slots, states.to(DEV), om, ph, proj.tau_star_inv)
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    s_own, s_ws = states.to(DEV), states.to(DEV)
    for _ in range(2):
        y_own = ops.ragged_step(dq, dk, dv, db, dl, cu, slots, s_own, om, ph, proj.tau_star_inv)
        y_ws = ops.ragged_step(dq, dk, dv, db, dl, cu, slots, s_ws, om, ph, proj.tau_star_inv, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(y_own, y_ws)
        assert torch.equal(s_own, s_ws)
    with pytest.raises(ValueError):
        ops.ragged_workspace_bytes(dq, dk, dv, db, dl, [0, 1], slots, s_ws, om, ph, proj.tau_star_inv)


def test_padding_and_out_of_range_device_slots_are_skipped(proj, oproj):
    """Device slots are not checked on the host (that would synchronise): a negative slot (padding) and a
    slot past the slab are skipped on the device -- their states untouched, their y rows left as they
    were -- while the other sequences match the oracle."""
    lens = [1, 1, 45, 1, 70, 1, 9]
    n_slots = 10
    q, k, v, beta, lam, cu, slots, states = make_step(lens, 2, 64, torch.float32, n_slots, seed=8)
    bad = {1: -1, 4: n_slots + 3, 6: -7}          # decode padding, prefill past the slab, prefill padding
    for i, s in bad.items():
        slots[i] = s
    sd = states.to(DEV)
    y = torch.full((q.shape[0], 2, 64), 123.0, device=DEV)
    ops.ragged_step(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), cu, slots.to(DEV), sd,
                    proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv, y=y,
                    cu_seqlens_device=cu.to(DEV))
    torch.cuda.synchronize()
    # the oracle over the other sequences only
    good = [i for i in range(len(lens)) if i not in bad]
    keep = torch.tensor(good)
    sub_cu, rows = [0], []
    for i in good:
        rows += list(range(int(cu[i]), int(cu[i + 1])))
        sub_cu.append(sub_cu[-1] + lens[i])
    rows_t = torch.tensor(rows)
    Yr, Sr = oracle_step(q[rows_t], k[rows_t], v[rows_t], beta[rows_t], lam[rows_t], torch.tensor(sub_cu),
                         slots[keep], states, oproj)
    yc = y.cpu()
    assert rel_l2(yc[rows_t].numpy(), Yr) < 1e-4
    for i in bad:
        assert bool((yc[int(cu[i]):int(cu[i + 1])] == 123.0).all()), i
    used = set(int(slots[i]) for i in good)
    S = sd.cpu()
    for s in range(n_slots):
        if s in used:
            assert rel_l2(S[s].numpy(), Sr[s]) < 1e-4, s
        else:
            assert torch.equal(S[s], states[s]), s
    with pytest.raises(ValueError, match="outside"):   # the same slots from the host are rejected
        ops.ragged_step(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), cu, slots, sd,
                        proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv)


@pytest.mark.parametrize("gather_slots", [False, True])
def test_serving_op_without_host_sync(proj, oproj, gather_slots):
    """hybrid_recurrent_forward with the scheduler's host offsets, their device copy and device slots (or
    slots gathered from slot_mapping on the device): one step under torch's sync debug mode "error" (any
    synchronising call or blocking copy raises), with results equal to the oracle's."""
    lens = [1, 40, 1, 1, 25, 0]
    q, k, v, beta, lam, cu, slots, states = make_step(lens, 2, 64, torch.float32, 9, seed=12)
    slot_mapping = torch.repeat_interleave(slots.to(torch.int64), torch.tensor(lens)).to(DEV)
    rs = states.transpose(2, 3).contiguous().to(DEV)
    qd, kd, vd, bd, ld = (t.to(DEV) for t in (q, k, v, beta, lam))
    cu_d, slots_d = cu.to(DEV), slots.to(DEV)
    out = torch.empty(q.shape[0], 2, 64, device=DEV)
    ws = torch.empty(ops.ragged_workspace_bytes(qd, kd, vd, bd, ld, cu, slots_d, rs.transpose(2, 3),
                                                proj.device_omega(DEV), proj.device_phase(DEV), proj.tau_star_inv),
                     dtype=torch.uint8, device=DEV)
    kw = dict(cu_seqlens=cu, cu_seqlens_device=cu_d, seq_slots=None if gather_slots else slots_d, fwht_proj=proj,
              workspace=ws)
    scratch = rs.clone()
    hybrid_recurrent_forward(qd, kd, vd, bd, ld, scratch, slot_mapping, out, **kw)   # first call: streams, tables
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        hybrid_recurrent_forward(qd, kd, vd, bd, ld, rs, slot_mapping, out, **kw)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    Yr, Sr = oracle_step(q, k, v, beta, lam, cu, slots, states, oproj)
    assert rel_l2(out.cpu().numpy(), Yr) < 1e-4
    for i, s in enumerate(slots.tolist()):
        if lens[i]:
            assert rel_l2(rs[s].transpose(1, 2).cpu().numpy(), Sr[s]) < 1e-4


def _slot_map(lens, slots):
    return torch.repeat_interleave(torch.as_tensor(slots, dtype=torch.int64), torch.tensor(lens))


def test_reference_signature_without_host_sync(proj, oproj):
    """hybrid_recurrent_forward with the reference op's eight arguments only (kdn_slot_step: runs, split and
    packed prefill layout on the device) under torch's sync debug mode "error": decodes, prefills of 2, 64,
    300 and 64 * 140 + 17 tokens (the last spans two 128-slot windows), padding runs; results against the
    float64 oracle, slots no run uses bit-identical."""
    lens = [1, 2, 1, 300, 5, 1, 64 * 140 + 17, 64, 1]
    run_slots = [3, 7, -1, 0, -1, 11, 5, 2, 9]          # -1: padding runs
    H, n_slots = 2, 12
    g = torch.Generator().manual_seed(21)
    T = int(sum(lens))
    q = torch.randn(T, H, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(T, H, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(T, H, 64, generator=g).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(T, H, generator=g))
    lam = 0.95 + 0.05 * torch.rand(T, H, generator=g)
    states = 0.05 * torch.randn(n_slots, H, 512, 64, generator=g)
    slot_mapping = _slot_map(lens, run_slots).to(DEV)
    qd, kd, vd, bd, ld = (t.to(DEV) for t in (q, k, v, beta, lam))
    out = torch.full((T, H, 64), 7.0, device=DEV, dtype=torch.bfloat16)
    scratch = states.transpose(2, 3).contiguous().to(DEV)
    hybrid_recurrent_forward(qd, kd, vd, bd, ld, scratch, slot_mapping, out)   # first call: tables, streams
    torch.cuda.synchronize()
    rs = states.transpose(2, 3).contiguous().to(DEV)
    out.fill_(7.0)
    torch.cuda.set_sync_debug_mode("error")
    try:
        hybrid_recurrent_forward(qd, kd, vd, bd, ld, rs, slot_mapping, out)
    finally:
        torch.cuda.set_sync_debug_mode("default")
    torch.cuda.synchronize()
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int64)
    live = [i for i, s in enumerate(run_slots) if s >= 0]
    y = out.float().cpu().numpy()
    S = rs.transpose(2, 3).cpu()
    for i in live:
        lo, hi, s = int(cu[i]), int(cu[i + 1]), run_slots[i]
        for h in range(H):
            pq = ol.lift(q[lo:hi, h].float().numpy(), oproj)
            pk = ol.lift(k[lo:hi, h].float().numpy(), oproj)
            yr, Sr = osc.token_recurrence(pq[None], pk[None], v[lo:hi, h].double().numpy()[None],
                                          beta[lo:hi, h].double().numpy()[None], lam[lo:hi, h].double().numpy()[None],
                                          states[s, h].double().numpy().T[None])
            assert rel_l2(y[lo:hi, h], yr[0]) < TOL[torch.bfloat16], (i, h)
            assert rel_l2(S[s, h].numpy(), Sr[0].T) < TOL[torch.bfloat16], (i, h)
    for i, s in enumerate(run_slots):   # padding rows keep what the caller had
        if s < 0:
            assert (out[int(cu[i]):int(cu[i + 1])].float() == 7.0).all()
    used = {s for s in run_slots if s >= 0}
    for s in range(n_slots):
        if s not in used:
            assert torch.equal(S[s], states[s]), s


@pytest.mark.parametrize("dtype,schedule", [(torch.float32, "split"), (torch.bfloat16, "split"),
                                            (torch.bfloat16, "fused")])
def test_slot_step_equals_ragged_step(proj, monkeypatch, dtype, schedule):
    """kdn_slot_step (layout from the slot map on the device, packed windows) against kdn_ragged_step (host
    offsets, segments) on the same step, both on one schedule: the same kernels and products, so y and the
    states agree bit for bit."""
    monkeypatch.setenv("KDN_SCAN_SCHEDULE", schedule)
    lens = [1, 37, 1, 200, 1, 64, 130, 1, 2, 64 * 130 + 5]
    q, k, v, beta, lam, cu, slots, states = make_step(lens, 2, 64, dtype, 16, seed=23)
    d = lambda t: t.to(DEV)
    s1, s2 = d(states), d(states)
    y1 = ops.ragged_step(d(q), d(k), d(v), d(beta), d(lam), cu, slots, s1, proj.device_omega(DEV),
                         proj.device_phase(DEV), proj.tau_star_inv)
    y2 = ops.slot_step(d(q), d(k), d(v), d(beta), d(lam), d(_slot_map(lens, slots)), s2, proj.device_omega(DEV),
                       proj.device_phase(DEV), proj.tau_star_inv)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert torch.equal(s1, s2)


def test_slot_step_rejects_maps_with_too_many_runs(proj):
    """2 slots allow at most 5 runs: a map of 7 alternating runs is invalid, status is set to 1 and nothing
    runs (states and y untouched)."""
    lens = [3, 1, 4, 1, 5, 1, 2]
    q, k, v, beta, lam, _, _, states = make_step(lens, 2, 64, torch.float32, 2, seed=5)
    sm = _slot_map(lens, [0, 1, 0, 1, 0, 1, 0]).to(torch.int32).to(DEV)
    sd = states.to(DEV)
    y = torch.full((q.shape[0], 2, 64), 3.0, device=DEV)
    status = torch.zeros(1, dtype=torch.int32, device=DEV)
    ops.slot_step(q.to(DEV), k.to(DEV), v.to(DEV), beta.to(DEV), lam.to(DEV), sm, sd, proj.device_omega(DEV),
                  proj.device_phase(DEV), proj.tau_star_inv, y=y, status=status)
    torch.cuda.synchronize()
    assert int(status[0]) == 1
    assert torch.equal(sd.cpu(), states) and (y == 3.0).all()
