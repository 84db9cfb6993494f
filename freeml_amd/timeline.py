"""Per-workgroup timelines of the grouped decode kernel.

With FMLH_GROUPED_TRACE=<file> set when an engine is created, every grouped decode launch
appends to <file> a header {steps, workgroups, points, n_layer} and the device wall clock
(100 MHz ticks) at each trace point of its first `steps` decode steps, for each of the first
`workgroups` workgroups (decode_grouped_kernel.h, `stamp`).  Slot 0 is the step start, slot
1 + 16 l + k is point k of layer l (below), and 1 + 16 L + 0 / 1 close the lm_head products and
the token pick.  Each interval is the time from the previous point to this one.
"""
import numpy as np

# Point k of a layer closes the interval named here (what the workgroup did since point k-1).
POINTS = [
    ("ln0", "wait for the previous layer's dx2 words, x += dx2, LayerNorm 0"),
    ("qkv", "QKV rows on matrix cores"),
    ("att_wait", "emit q / k_new / v_new, request cached K/V rows, wait for the item's q/k/v"),
    ("att", "attention of the workgroup's items"),
    ("att_emit", "combine the waves, emit y"),
    ("y_wait", "wait for / gather all y words"),
    ("proj", "attention projection rows on matrix cores"),
    ("proj_emit", "emit dx1, request W_proj2 slice"),
    ("ln1", "wait for dx1 words, x += dx1, LayerNorm 1"),
    ("fc", "FC rows on matrix cores"),
    ("gelu", "GELU into the workgroup's h slice"),
    ("proj2", "proj2 partial of every output over the h slice, matrix cores"),
    ("stage", "stage the partials in LDS"),
    ("part_emit", "emit the partials, request the next W_qkv slice"),
    ("part_wait", "wait for / gather the partials of the workgroup's outputs"),
    ("dx2_emit", "sum the partials, emit dx2"),
]
PER_LAYER = len(POINTS)
TICK_US = 0.01  # 100 MHz


def read(path):
    """Launches in the file: a list of (array [steps][workgroups][points] of ticks, n_layer)."""
    raw = np.fromfile(path, dtype=np.uint64)
    out, i = [], 0
    while i + 4 <= raw.size:
        steps, wgs, pts, n_layer = (int(x) for x in raw[i:i + 4])
        n = steps * wgs * pts
        out.append((raw[i + 4:i + 4 + n].reshape(steps, wgs, pts).astype(np.int64), n_layer))
        i += 4 + n
    return out


def summarize(trace, n_layer, step=1, workgroups=None):
    """Mean over workgroups (those that stamped) of each interval of one decode step, in us,
    summed over the layers, plus the lm_head intervals and the step total."""
    t = trace[step]
    wg = np.arange(t.shape[0]) if workgroups is None else np.arange(workgroups)
    t = t[wg]
    live = t[:, 0] > 0
    t = t[live]
    res, prev = {}, t[:, 0]
    for l in range(n_layer):
        for k, (name, _) in enumerate(POINTS):
            cur = t[:, 1 + PER_LAYER * l + k]
            res[name] = res.get(name, 0.0) + float(np.mean(cur - prev)) * TICK_US
            prev = cur
    lm = t[:, 1 + PER_LAYER * n_layer]
    pick = t[:, 2 + PER_LAYER * n_layer]
    res["lm_head"] = float(np.mean(lm - prev)) * TICK_US
    res["pick"] = float(np.mean(pick - lm)) * TICK_US
    res["step"] = float(np.mean(pick - t[:, 0])) * TICK_US
    res["workgroups"] = int(live.sum())
    return res
