"""CPU model of the LDS-DMA tile kernel's transfer schedule (mfma_dma_kernel.hpp).

The kernel's producers issue global->LDS transfers that the compiler does not
see; one explicit `s_waitcnt vmcnt(N)` per iteration is all that orders them
against the LDS reads.  This model replays the producer loop's control (the
same ring counters, lookaheads and wait count as the kernel) with in-order
retirement of a wavefront's transfers, and checks every LDS read of the
pipeline:
  * the producer's read of B row offsets from blocks(i + LB) (written by other
    producers: must have landed before the barrier that precedes the read),
  * the producer's scatter read of its own blocks(i + 1),
  * the consumers' read of B(i) after the barrier ending iteration i - 1,
and that no transfer in flight targets a slot that is read or re-targeted.
The wait count and ring sizes below restate the kernel's; a change to one
must be made to both."""
import pytest

KS = 4  # steps per iteration


def kernel_shape(kslots):
    lb = 3 if kslots == 1 else 2
    le = lb + 2
    nb, ne = lb + 1, le
    kops = kslots + KS
    kwait = KS + kops if lb == 3 else kops
    return lb, le, nb, ne, kops, kwait


def replay(kslots, niters, kwait=None, zero_prologue_b=True):
    """Returns the list of schedule violations (empty when the schedule is sound)."""
    lb, le, nb, ne, kops, kw = kernel_shape(kslots)
    kwait = kw if kwait is None else kwait
    bslot_of, eslot_of = {}, {}  # landed content per slot
    inflight = []                # (ring, slot, content) in issue order
    errors = []

    def read(ring, slot, content, who, it):
        held = (bslot_of if ring == "B" else eslot_of).get(slot)
        if held != content:
            errors.append(f"iter {it}: {who} expects {ring}{content} in slot {slot}, slot holds {held}")
        if any(r == ring and s == slot for r, s, _ in inflight):
            errors.append(f"iter {it}: {who} reads {ring} slot {slot} with a transfer to it in flight")

    def issue(ring, slot, content, count, it):
        if any(r == ring and s == slot for r, s, _ in inflight):
            errors.append(f"iter {it}: {ring} slot {slot} re-targeted with a transfer to it in flight")
        inflight.extend([(ring, slot, content)] * count)

    # kernel counters
    bslot = nb - 2 if zero_prologue_b else 0
    eslot = 0
    cons_bslot = 0
    for i in range(-le, niters):
        # packed blocks(i + LE) into eslot
        assert eslot == (i + le) % ne
        issue("E", eslot, i + le, kslots, i)
        # B(i + LB) into bslot, row offsets from blocks(i + LB) in slot em
        em = eslot - (le - lb) if eslot >= le - lb else eslot + lb
        assert em == (i + lb) % ne
        if i + lb >= 0:
            read("E", em, i + lb, "producer row-offset read", i)
        if i + lb >= 0 or zero_prologue_b:
            assert bslot == (i + lb) % nb
            issue("B", bslot, i + lb, KS, i)
            bslot = 0 if bslot == nb - 1 else bslot + 1
        # scatter of A(i + 1) from blocks(i + 1) in slot er
        if i + 1 >= 0:
            er = eslot + 1 - (ne if eslot + 1 >= ne else 0)
            assert er == (i + 1) % ne
            read("E", er, i + 1, "producer scatter read", i)
        # s_waitcnt vmcnt(kwait): all but the last kwait transfers have landed
        keep = inflight[len(inflight) - kwait:] if kwait else []
        for ring, slot, content in inflight[:len(inflight) - len(keep)]:
            (bslot_of if ring == "B" else eslot_of)[slot] = content
        inflight[:] = keep
        eslot = 0 if eslot == ne - 1 else eslot + 1
        # barrier; the consumers of iteration i + 1 read B(i + 1)
        if 0 <= i + 1 < niters:
            assert cons_bslot == (i + 1) % nb
            read("B", cons_bslot, i + 1, "consumer B read", i + 1)
            cons_bslot = 0 if cons_bslot == nb - 1 else cons_bslot + 1
    return errors


@pytest.mark.parametrize("kslots", [1, 2])
@pytest.mark.parametrize("niters", [1, 2, 3, 4, 7, 32])
def test_dma_schedule_every_read_sees_landed_data(kslots, niters):
    assert replay(kslots, niters) == []


def test_dma_schedule_model_catches_a_short_wait():
    """The model is not vacuous: a wait that lets one more transfer stay in
    flight, or a prologue without its zero B transfers, breaks it."""
    lb, le, nb, ne, kops, kwait = kernel_shape(1)
    assert replay(1, 8, kwait=kwait + 1)
    assert replay(1, 8, zero_prologue_b=False)
    assert replay(2, 8, kwait=kernel_shape(2)[5] + 1)


def test_dma_kernel_lds_budget():
    """Ring sizes of both slot counts fit the 160 KiB of LDS of a gfx950 CU."""
    for kslots in (1, 2):
        lb, le, nb, ne, kops, kwait = kernel_shape(kslots)
        b = nb * KS * 32 * 64 * 2          # B tiles, 32 rows x 64 halves per step
        e = ne * KS * 256 * kslots * 4     # packed blocks
        a = KS * 2 * (128 * 32 + 64) * 2   # A tiles (2 slots per step), one dummy cell per lane
        assert b + e + a <= 160 * 1024
        assert kwait + kops <= 63          # vmcnt range
