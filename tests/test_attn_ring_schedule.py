"""The attention kernel's K / V ring schedule (csrc/attn.hip, attn_fwd_kernel), checked as a model on the CPU.

Per q tile the kernel copies K(0..2) and V(0..1) into slots 0..2 / 0..1, waits for them, synchronises the
workgroup, computes QK(0) from K slot 0, then runs steps t = 0 .. nkt-2: step t copies K(t+3) into slot
(t+3) % 4 and V(t+2) into slot (t+2) % 4 (tiles clamped to nkt-1), computes QK(t+1) from K slot (t+1) % 4
and PV(t) from V slot t % 4; after the steps, PV(nkt-1) reads V slot (nkt-1) % 4.  A workgroup barrier,
preceded by a wait for the wave's own copies, follows every even step.  The waves of a workgroup run
unsynchronised between barriers, so the schedule is race-free only if

* every read finds the tile it wants in its slot, copied behind a barrier (copy step <= x <= read step - 1
  for some barrier after step x), and
* no slot is refilled before every wave has finished reading the tile in it (a barrier after some step x
  with read step <= x <= refill step - 1).

The same model flags the schedule with the barrier after every odd step instead: there a wave could start
step 1, whose copy refills K(0)'s slot, while another was still computing QK(0).
"""

NK = NV = 4


def ring_events(nkt: int, barrier_parity: int):
    """(step, 'w' | 'r', ring, tile, slot) in program order, and the steps followed by a barrier."""
    ev = [(-2, "w", "K", min(k, nkt - 1), k) for k in range(3)]
    ev += [(-2, "w", "V", min(k, nkt - 1), k) for k in range(2)]
    ev.append((-1, "r", "K", 0, 0))
    bars = {-2, nkt - 1}                  # after the prologue copies; after the last PV
    for t in range(nkt - 1):
        ev.append((t, "w", "K", min(t + 3, nkt - 1), (t + 3) % NK))
        ev.append((t, "w", "V", min(t + 2, nkt - 1), (t + 2) % NV))
        ev.append((t, "r", "K", t + 1, (t + 1) % NK))
        ev.append((t, "r", "V", t, t % NV))
        if t % 2 == barrier_parity:
            bars.add(t)
    ev.append((nkt - 1, "r", "V", nkt - 1, (nkt - 1) % NV))
    return ev, bars


def ring_errors(nkt: int, barrier_parity: int):
    ev, bars = ring_events(nkt, barrier_parity)

    def barrier_between(a, b):
        return any(a <= x <= b for x in bars)

    errs = []
    for ring in ("K", "V"):
        writes = [(st, i, tile, slot) for i, (st, kd, rg, tile, slot) in enumerate(ev) if kd == "w" and rg == ring]
        reads = [(st, tile, slot) for st, kd, rg, tile, slot in ev if kd == "r" and rg == ring]
        for rst, tile, slot in reads:
            src = [w for w in writes if w[3] == slot and w[0] < rst]
            if not src or src[-1][2] != tile:
                errs.append(f"{ring}{tile} not in slot {slot} at step {rst}")
                continue
            wst, wi = src[-1][0], src[-1][1]
            if not barrier_between(wst, rst - 1):
                errs.append(f"{ring}{tile} read at step {rst}: its copy (step {wst}) is not behind a barrier")
            for w2 in writes:
                if w2[3] == slot and w2[1] > wi and not barrier_between(rst, w2[0] - 1):
                    errs.append(f"{ring}{tile} read at step {rst} races the refill of slot {slot} at step {w2[0]}")
    return errs


def test_ring_schedule_race_free():
    """Every key-tile count a q tile can have at S <= 16384 (nkt = 1 .. 256), and samples up to S = 65536:
    no read misses its tile and no slot is refilled under a read.  The steady schedule repeats every two
    steps (four ring slots, one barrier), so the prologue, the tail cases of both step parities and a
    few periods cover every length."""
    for nkt in list(range(1, 257)) + [300, 511, 512, 513, 1023, 1024]:
        assert ring_errors(nkt, barrier_parity=0) == [], nkt


def test_ring_model_flags_odd_step_barriers():
    """The model is not vacuous: with barriers after the odd steps, step 1's refill of K(0)'s slot races the
    QK(0) before the loop for every q tile with three or more key tiles."""
    flagged = [nkt for nkt in range(1, 64) if ring_errors(nkt, barrier_parity=1)]
    assert flagged == list(range(3, 64))
    assert any("K0 read at step -1 races" in e for e in ring_errors(10, barrier_parity=1))
