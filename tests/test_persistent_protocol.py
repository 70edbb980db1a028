"""The persistent kernel's synchronisation protocol, replayed on the CPU for every
workgroup of many grids: both wavefront roles execute the same barrier sequence
(a mismatch would hang the workgroup), every K tile is in LDS before the compute
waves read it, no ring stage is overwritten while it is being read, and a loader
never has more loads in flight than the 6-bit vmcnt counter holds.

The replay follows the control flow of gemmMfmaPersistentKernel
(ridge_amd/csrc/gemm_mfma.hpp) statement for statement: the tile count of each
workgroup, the loader's prologue, issue and wait schedule and the compute waves'
barrier and read schedule. Loads complete in issue order (the vmcnt semantics
the kernel relies on)."""
import itertools

import pytest

from ridge_amd import gemm as G


def _traits(v):
    loaders = 2
    la = v.BM * v.BK * 2 // 1024 // loaders
    lb = v.BK * v.BN * 2 // 1024 // loaders
    return la, lb


def replay(v, M, N, K, grid, self, wait_slack=0):
    """Returns the barrier sequence both roles execute and raises on a hazard.
    wait_slack > 0 plants a mistake: every steady-state wait allows that many
    more loads in flight than the kernel's."""
    BM, BN, BK, S = v.BM, v.BN, v.BK, v.stages
    LA, LB = _traits(v)
    L = LA + LB  # loads per K tile and loader
    num_tiles = (M // BM) * (N // BN)
    num_k = K // BK
    G_ = ((num_tiles - self + grid - 1) // grid) * num_k

    queue = []          # in-flight loads in issue order: [stage, ktile, part, loads]
    stages = {}         # stage -> (ktile, landed epoch or None)
    issued_at = set()   # (stage, epoch) of every refill
    landed = {}         # epoch -> snapshot of stages (what compute may read in it)
    epoch = 0

    def issue(stage, ktile):
        # The A loads of a K tile are issued before its B loads.
        stages[stage] = (ktile, None)
        queue.append([stage, ktile, "A", LA])
        queue.append([stage, ktile, "B", LB])
        issued_at.add((stage, epoch))
        assert sum(q[3] for q in queue) <= 63, "vmcnt overflow"

    def wait(n):
        while sum(q[3] for q in queue) > n:
            stage, ktile, part, _ = queue.pop(0)
            if part == "B" and stages[stage][0] == ktile:
                stages[stage] = (ktile, epoch)

    lbar = []

    def barrier(label):
        nonlocal epoch
        lbar.append(label)
        epoch += 1
        landed[epoch] = dict(stages)

    # Loader: prologue, then one refill per K tile.
    for s_ in range(S - 1):
        if s_ < G_:
            issue(s_, s_)
    wait((S - 2) * L if G_ >= S - 1 else 0)
    barrier("B0")
    for g in range(G_ - 1):
        if g + S - 1 < G_:
            issue((g + S - 1) % S, g + S - 1)
            wait((S - 2) * L + wait_slack)
        else:
            wait(0)
        barrier("B%d" % (g + 1))

    # Compute: reads K tile g right after B_g (its later k-steps in the same epoch).
    cbar = []

    def read(ktile, ep):
        stage = ktile % S
        held, when = landed[ep].get(stage, (None, None))
        assert held == ktile and when is not None and when < ep, \
            "K tile %d read from stage %d before it landed (holds %s)" % (ktile, stage, held)
        assert (stage, ep) not in issued_at, "stage %d overwritten while K tile %d is read" % (stage, ktile)

    cbar.append("B0")
    read(0, 1)
    for g in range(G_):
        if g + 1 < G_:
            cbar.append("B%d" % (g + 1))
            read(g + 1, len(cbar))
    assert lbar == cbar, "barrier sequences differ"
    return lbar


def _persistent_rows():
    return [v for v in G.variants() if v.schedule == 2]


SHAPES = [(m, n, k) for m, n, k in itertools.product((256, 768, 2048, 8192), (128, 384, 1024, 8192),
                                                          (32, 64, 128, 192, 256, 448, 1024))]


@pytest.mark.parametrize("v", _persistent_rows(), ids=lambda v: v.label())
def test_persistent_protocol_every_workgroup(v):
    checked = 0
    for (M, N, K) in SHAPES + [(8192, 8192, 128), (16384, 128, 8192), (4096, 4096, 4096), (37 * v.BM, 11 * v.BN, 3 * v.BK)]:
        if M % v.BM or N % v.BN or K % v.BK:
            continue
        tiles = (M // v.BM) * (N // v.BN)
        for grid in sorted({min(tiles, 256), min(tiles, 7), min(tiles, 100)}):
            for self in range(grid):
                replay(v, M, N, K, grid, self)
                checked += 1
    assert checked > 1000


def test_replay_catches_a_planted_mistake():
    """The replay is a checker: a loader whose steady-state wait lets one more K
    tile stay in flight than the kernel's lets the compute waves read it early."""
    v = [w for w in _persistent_rows() if w.BM == 128 and w.BN == 128][0]
    LA, LB = _traits(v)
    replay(v, 8192, 8192, 1024, 256, 0)  # the kernel's own waits: clean
    with pytest.raises(AssertionError, match="before it landed"):
        replay(v, 8192, 8192, 1024, 256, 0, wait_slack=LB)
