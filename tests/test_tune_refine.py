"""tune.refine on the host: which rows it re-times and how it rewrites the
timing CSV (the GPU timing itself is replaced by a script)."""
import csv

from tilec import tune

ROWS = [
    # shape A: two configs within 10 % of the best, one far behind
    ("16", "4096", "4096", "f32", "0", "skinny_f32_w4_b1", "64", "1", "15.36"),
    ("16", "4096", "4096", "f32", "0", "skinny_f32_w4_b2", "64", "1", "14.855"),
    ("16", "4096", "4096", "f32", "0", "gemm_f32_64x64x16_w2x2", "64", "1", "40.0"),
    # shape B: a single config
    ("64", "64", "64", "f32", "0", "gemm_f32_64x64x16_w2x2", "64", "1", "0.5"),
]


def write(path):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(tune.FIELDS)
        for M, K, N, dt, lay, kern, bn, split, ms in ROWS:
            w.writerow(["gfx950", "256", M, K, N, dt, lay, kern, "16", bn, "1024", split, ms])


def test_refine_retimes_close_configs_and_keeps_medians(tmp_path, monkeypatch):
    path = tmp_path / "t.csv"
    write(path)
    new = {"skinny_f32_w4_b1": [14.6, 14.5, 14.7], "skinny_f32_w4_b2": [14.9, 15.0, 14.8]}
    calls = []

    def fake_time(x1, x2, cfg, best=None, reps=5, x2s=None):
        calls.append(cfg)
        return new[cfg[0]][sum(c == cfg for c in calls) - 1]

    monkeypatch.setattr(tune, "operands", lambda *a: (None, None))
    monkeypatch.setattr(tune, "operands_for", lambda *a: [None])
    monkeypatch.setattr(tune, "settle", lambda *a, **k: None)
    monkeypatch.setattr(tune, "time_ms", fake_time)
    tune.refine(path=str(path), rounds=3, gen=object())
    # only the two close configs of shape A, three passes, alternating order
    assert calls == [("skinny_f32_w4_b2", 1), ("skinny_f32_w4_b1", 1), ("skinny_f32_w4_b1", 1),
                     ("skinny_f32_w4_b2", 1), ("skinny_f32_w4_b2", 1), ("skinny_f32_w4_b1", 1)]
    with open(path) as f:
        out = list(csv.DictReader(f))
    assert list(out[0].keys()) == tune.FIELDS and len(out) == len(ROWS)
    ms = [float(r["ms"]) for r in out]
    assert ms[0] == 14.65  # median of 15.36, 14.6, 14.5, 14.7: (14.6 + 14.7) / 2
    assert ms[1] == 14.8775  # median of 14.855, 14.9, 15.0, 14.8: (14.855 + 14.9) / 2
    assert ms[2:] == [40.0, 0.5]  # far behind, or alone: untouched
    assert [r["kernel"] for r in out] == [r[5] for r in ROWS]
