"""The relay timeline reader and summary (freeml_amd/timeline.py) on a synthetic trace whose
intervals are known: the file layout the library writes (a 10-word header, then
[step][role][point] ticks of 100 MHz) and the per-layer path of sequence 0."""
import numpy as np

from freeml_amd import timeline


def _trace(steps=4, L=2, nq=1, H=1, nf=2, nf2=0, n_a=1, nlm=1, points=8):
    per = nq + n_a * H + nf + nf2
    roles = L * per + nlm
    t = np.zeros((steps, roles, points), dtype=np.uint64)
    for s in range(steps):
        base = 1000 * s
        for l in range(L):
            o, b = l * per, base + 100 * l
            t[s, o, 1], t[s, o, 3] = b + 5, b + 8                   # Q
            a = o + nq
            t[s, a, 1], t[s, a, 3] = b + 10, b + 40                 # A: in, dx1 out
            for k, skew in enumerate((0, 3)):                     # F: the second member is 3 ticks later
                f = o + nq + n_a * H + k
                t[s, f, 1], t[s, f, 3], t[s, f, 4] = b + 50 + skew, b + 70 + skew, b + 87 + skew
            for r in range(o, o + per):
                t[s, r, 6], t[s, r, 7] = 300, 20 + r
        lm = L * per
        t[s, lm, 5], t[s, lm, 6], t[s, lm, 7] = base + 500, 900, 100
    hdr = np.array([steps, roles, points, L, nq, H, nf, nf2, n_a, nlm], dtype=np.uint64)
    return np.concatenate([hdr, t.ravel()])


def test_relay_summary_reads_the_layout_and_the_critical_members(tmp_path):
    path = tmp_path / "trace.bin"
    np.concatenate([_trace(), _trace()]).tofile(path)  # two launches, appended
    launches = timeline.read_relay(str(path))
    assert len(launches) == 2
    trace, meta = launches[-1]
    assert trace.shape == (4, 9, 8)
    assert meta == dict(n_layer=2, nq=1, n_head=1, nf=2, nf2=0, nA=1, nlm=1)
    r = timeline.summarize_relay(trace, meta)
    c = {k: round(v, 6) for k, v in r["chain"].items()}
    # Layer 1: x_1 complete at the later FC member's rows (90), A in 110 .. out 140, F in 153
    # (the later member) .. out 173, rows 190.
    assert c == {"x_to_A": 0.2, "A": 0.3, "A_to_F": 0.13, "F": 0.2, "F_to_rows": 0.17, "layer": 1.0}
    assert abs(r["step_us"] - 10.0) < 1e-9
    assert abs(r["teams"]["lm"]["wait"] - 9.0) < 1e-9 and abs(r["teams"]["lm"]["busy"] - 1.0) < 1e-9
    assert abs(r["teams"]["Q"]["wait"] - 3.0) < 1e-9
    # Q roles are 0 and 4: busy ticks 20 and 24, mean 22.
    assert abs(r["teams"]["Q"]["busy"] - 0.22) < 1e-9
