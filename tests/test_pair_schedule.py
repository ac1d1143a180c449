"""CPU model of the paired tile kernel's pipeline (mfma_pair_kernel.hpp).

Consumer w reads the fragments of tile i + 1 during iteration i and runs the
MFMAs of tile i; staging wavefront w writes tile i + 2 into slot (i + 2) & 1
during iteration i from data it loaded in iteration i - 2, and clears the
cells of the tile that held the slot before.  One barrier ends each
iteration.  This model replays both loops over the same iteration range and
checks, for every tile, that (1) the slot holds exactly that tile when the
consumer reads it (written in an earlier iteration, not overwritten before
the read, previous occupant's cells cleared), (2) every load is issued
before the iteration that uses its data, and (3) both roles pass the same
number of barriers.  The constants restate the kernel's; a change to one
must be made to both."""
import pytest

KS = 4            # steps per iteration
FIRST = -4        # first loop iteration of both roles
SLOTS = 2         # A and B slots per consumer
WRITE_AHEAD = 2   # staging writes tile i + 2 in iteration i
DATA_AHEAD = 4    # ... loads the data of tile i + 4
UCOLS_AHEAD = 5   # ... the B-row offsets of tile i + 5
META_AHEAD = 6    # ... the entry range of tile i + 6
PRELOADED = {"ucols": [0], "meta": [0, 1]}


def replay(nsteps, w, write_ahead=WRITE_AHEAD, slots=SLOTS, data_ahead=DATA_AHEAD):
    niters = (nsteps + KS - 1) // KS
    valid = lambda n: 0 <= n and KS * n + w < nsteps
    errors = []
    slot = {}          # slot -> tile it holds (cells of that tile set)
    loaded = {"ucols": {n: -10**9 for n in PRELOADED["ucols"]},
              "meta": {n: -10**9 for n in PRELOADED["meta"]}, "data": {}}
    reads = []
    barriers = {"consumer": 0, "staging": 0}
    for i in range(FIRST, niters):
        # consumer part of iteration i: read tile i + 1 (if its step exists)
        n = i + 1
        if i >= -1 and valid(n) and (i == -1 or valid(i)):
            held = slot.get(n % slots)
            if held != n:
                errors.append(f"iter {i}: consumer reads slot {n % slots} holding {held}, expected tile {n}")
            reads.append(n)
        barriers["consumer"] += 1
        # staging part of iteration i
        t = i + write_ahead
        if valid(t):
            if loaded["data"].get(t, i) >= i:
                errors.append(f"iter {i}: tile {t} written from data not loaded in an earlier iteration")
            prev = slot.get(t % slots)
            if prev is not None and prev >= t:
                errors.append(f"iter {i}: tile {t} would replace newer tile {prev}")
            slot[t % slots] = t
        nu = i + UCOLS_AHEAD
        loaded["ucols"][nu] = i
        nd = i + data_ahead
        if loaded["ucols"].get(nd, i) >= i:
            errors.append(f"iter {i}: data of tile {nd} issued without its B-row offsets")
        if loaded["meta"].get(nd, i) >= i:
            errors.append(f"iter {i}: data of tile {nd} issued without its entry range")
        loaded["data"][nd] = i
        loaded["meta"][i + META_AHEAD] = i
        barriers["staging"] += 1
        # barrier: the consumer of iteration i + 1 reads tile i + 2 - 1 ... checked above
        # a slot may only be rewritten after its tile was read: the tile read in
        # iteration i is i + 1; the staging of iteration i wrote i + 2 into the
        # other slot, so the slot read next iteration must not be the one written now
        if valid(i + 2) and valid(i + 1) and (i + 2) % slots == (i + 1) % slots:
            errors.append(f"iter {i}: tile {i + 2} written into the slot of tile {i + 1} while it is read")
    expected = [n for n in range(niters) if valid(n)]
    if reads != expected:
        errors.append(f"consumer read tiles {reads}, expected {expected}")
    if barriers["consumer"] != barriers["staging"]:
        errors.append(f"barrier counts differ: {barriers}")
    return errors


@pytest.mark.parametrize("nsteps", [1, 2, 3, 4, 5, 7, 8, 9, 16, 33, 128, 131])
@pytest.mark.parametrize("w", range(KS))
def test_pair_schedule_every_read_sees_its_tile(nsteps, w):
    assert replay(nsteps, w) == []


def test_pair_schedule_model_catches_mistakes():
    """The model is not vacuous: writing one iteration later, a single slot,
    or loading data only one iteration ahead of the write break it."""
    assert any(replay(16, w, write_ahead=1) for w in range(KS))
    assert any(replay(16, w, slots=1) for w in range(KS))
    assert any(replay(16, w, data_ahead=2) for w in range(KS))


def test_pair_kernel_lds_budget():
    """A tiles (two slots per consumer, 64 dummy cells each), B tiles and,
    after the loop, the four partial tiles fit the 160 KiB of a gfx950 CU;
    every entry address fits the 16 bits of an entry word."""
    a_tile = (128 * 32 + 64) * 2
    a = KS * SLOTS * a_tile
    b = SLOTS * KS * 32 * 64 * 2
    red = KS * 32 * 64 * 16
    assert max(a + b, red) <= 160 * 1024
    assert (KS - 1) * 2 * a_tile + 2 * (128 * 32 + 63) < 65536
    # slot 1 is reached with the 16-bit immediate offset of ds_write
    assert a_tile < 65536
