"""The held-out sweep (registered in data/sweep/mi355x-heldout.md before it was
measured) scored against the model constants frozen with the registration:
the numbers reported for it, re-derived from the committed measurement."""
import os

import pytest

from ridge_amd import autotune as AT
from ridge_amd import tables as T
from ridge_amd import validate as V

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
MEASURED = os.path.join(ROOT, "data", "measured", "mi355x-heldout.csv")
REGISTERED = os.path.join(ROOT, "data", "sweep", "mi355x-heldout-registered.csv")
FROZEN = os.path.join(ROOT, "data", "sweep", "mi355x-heldout-hw.json")
IN_SAMPLE = os.path.join(ROOT, "data", "sweep", "mi355x-registered.csv")
# The kernel table at the registration commit; the held-out cross product is
# shapes x these rows, whatever the table holds now.
TABLE = os.path.join(ROOT, "data", "sweep", "mi355x-heldout-table.csv")


def test_heldout_shapes_are_disjoint_from_the_sweep_and_fully_measured():
    held = [s[:3] for s in T.read_shapes(REGISTERED)]
    assert len(held) == 14 and not set(held) & {s[:3] for s in T.read_shapes(IN_SAMPLE)}
    table = T.read(MEASURED)
    frozen = T.read(TABLE, require=V.KEY_COLUMNS)
    keys = [tuple(frozen.number(i, c, int) for c in V.KEY_COLUMNS) for i in range(len(frozen))]
    assert len(set(keys)) == 24
    absent, unexpected = V.registered_gate(table.records, T.read_shapes(REGISTERED), keys)
    assert not absent and not unexpected
    assert float(table.meta["canary_drift_fraction"]) <= 0.05


def test_heldout_accuracy_and_ranking_as_reported():
    rows = V.join(MEASURED, FROZEN)
    mape = sum(j.abs_pct for j in rows) / len(rows)
    assert mape == pytest.approx(10.35, abs=0.01)
    ranking = V.rank_shapes(rows)
    rhos = [s.rho for s in ranking]
    assert sum(rhos) / len(rhos) == pytest.approx(0.857, abs=0.001)
    assert max(s.regret1[0] for s in ranking) * 100 == pytest.approx(27.96, abs=0.01)


def test_heldout_pruning_as_reported():
    """k = 10 meets the <= 2% target exactly (14 of 14); k = 1 is worse than on
    the in-sample sweep but better than every model-free ranking."""
    table, total, shapes, _ = AT.evaluate(MEASURED, FROZEN, ks=(1, 2, 3, 10))
    by_k = {r["k"]: r for r in table}
    assert (total, shapes) == (336, 14)
    assert by_k[1]["mean_regret"] == pytest.approx(9.32, abs=0.01) and by_k[1]["hits"] == 3
    assert by_k[2]["mean_regret"] == pytest.approx(1.25, abs=0.01)
    assert by_k[10]["mean_regret"] == 0.0 and by_k[10]["hits"] == 14
    base = AT.baselines(MEASURED, FROZEN, ks=(1, 10))
    assert base[1]["random"][0] == pytest.approx(24.18, abs=0.01)
    assert all(by_k[1]["mean_regret"] < v[0] for v in base[1].values())
