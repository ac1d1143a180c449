"""CPU model of the LDS-DMA tile kernel's transfer schedule (mfma_dma_kernel.hpp).

The kernel's producers issue global->LDS transfers of B tiles that the
compiler does not see; one explicit `s_waitcnt vmcnt(N)` per iteration is all
that orders them against the consumers' LDS reads.  This model replays the
producer loop's control (the same ring counters, lookahead and wait count as
the kernel) with in-order retirement of a wavefront's transfers, and checks
that after the barrier ending iteration i the consumers' B(i + 1) has landed
and that no transfer in flight targets a slot that is read or re-targeted.
(The consumers' own entry loads are ordinary loads whose waits the compiler
places.)  The constants below restate the kernel's; a change to one must be
made to both."""
import pytest

KS = 4        # steps per iteration = transfers per producer and iteration
LB = 3        # B lookahead (iterations)
NB = LB + 1   # B ring slots
WAIT = (LB - 1) * KS


def replay(niters, wait=WAIT, lb=LB, nb=NB):
    """Returns the list of schedule violations (empty when the schedule is sound)."""
    landed = {}
    inflight = []  # (slot, content) in issue order
    errors = []
    bslot = 0        # producer: slot of B(i + lb)
    cons_bslot = 0   # consumer: slot of B(i)
    for i in range(-lb, niters):
        assert bslot == (i + lb) % nb
        if any(s == bslot for s, _ in inflight):
            errors.append(f"iter {i}: slot {bslot} re-targeted with a transfer to it in flight")
        if i >= 0 and bslot == cons_bslot:
            errors.append(f"iter {i}: B({i + lb}) written into the slot consumers read in this iteration")
        inflight.extend([(bslot, i + lb)] * KS)
        bslot = 0 if bslot == nb - 1 else bslot + 1
        keep = inflight[max(0, len(inflight) - wait):] if wait else []
        for slot, content in inflight[:len(inflight) - len(keep)]:
            landed[slot] = content
        inflight[:] = keep
        if i >= 0:
            cons_bslot = 0 if cons_bslot == nb - 1 else cons_bslot + 1
        # barrier; the consumers of iteration i + 1 read B(i + 1)
        if 0 <= i + 1 < niters:
            assert cons_bslot == (i + 1) % nb
            if landed.get(cons_bslot) != i + 1:
                errors.append(f"iter {i + 1}: consumers read slot {cons_bslot} holding {landed.get(cons_bslot)}, "
                              f"expected B({i + 1})")
            if any(s == cons_bslot for s, _ in inflight):
                errors.append(f"iter {i + 1}: consumers read slot {cons_bslot} with a transfer to it in flight")
    return errors


@pytest.mark.parametrize("niters", [1, 2, 3, 4, 7, 32, 33])
def test_dma_schedule_every_read_sees_landed_data(niters):
    assert replay(niters) == []


def test_dma_schedule_model_catches_a_short_wait_or_ring():
    """The model is not vacuous: a wait that leaves one more transfer in
    flight, or a ring one slot short, breaks it."""
    assert replay(8, wait=WAIT + 1)
    assert replay(8, nb=NB - 1)


def test_dma_kernel_lds_budget():
    """B ring and A tiles (and, after the loop, the four partial tiles) fit
    the 160 KiB of LDS of a gfx950 CU; the wait count fits vmcnt."""
    b = NB * KS * 32 * 64 * 2          # B tiles, 32 rows x 64 halves per step
    a = KS * 2 * (128 * 32 + 64) * 2   # A tiles (2 slots per step), one dummy cell per lane
    red = KS * 32 * 64 * 16            # partial 128 x 64 fp32 tiles
    assert max(b + a, red) <= 160 * 1024
    assert WAIT + KS <= 63
