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


# The wide decode kernel (decode_wide.h, WideArgs::trace): with FMLH_WIDE_TRACE=<file> set when
# an engine is created, every wide launch appends a header {workgroups, points, n_layer, batch}
# and, for every workgroup, the device wall clock (100 MHz ticks) at each point of its decode
# step 1: point k of layer l at 12 l + k, the lm_head's points at 12 L + k.  Point k closes the
# interval named here (what the workgroup did since the previous point).
WIDE_POINTS = [
    ("start", "close of the previous layer (or the step's embedding)"),
    ("ln0", "wait for the dx2 words (one proxy per producer, then every word), x += dx2, LayerNorm 0"),
    ("qkv", "QKV rows, emit q / k_new / v_new; request the projection rows"),
    ("att", "attention item: wait for q, stream the key slice's K/V rows, emit the record"),
    ("merge", "pair-merge workgroups: gather the pair's records in slice order, emit y"),
    ("y_in", "wait for / gather every y word"),
    ("proj", "projection rows, emit dx1; request the FC rows and the W_proj2 block"),
    ("dx1_in", "wait for / gather every dx1 word, x += dx1"),
    ("fc", "LayerNorm 1, FC rows + GELU, emit h words"),
    ("part", "gather the team's h words, MLP-projection partials of the member's outputs, emit"),
    ("part_in", "wait for / gather the owner's partials"),
    ("dx2", "sum the partials in team order, emit dx2"),
]
WIDE_LM = [("x_in", "wait for / gather the last dx2, x += dx2, ln_f"),
           ("logits", "lm_head rows (streamed one round ahead)"),
           ("cand", "first-maximum candidate of the workgroup's rows, emit"),
           ("tokens", "wait for / gather every candidate, pick the tokens")]


def read_wide(path):
    """Wide launches in the file: a list of (array [workgroups][points] of ticks, n_layer, batch)."""
    raw = np.fromfile(path, dtype=np.uint64)
    out, i = [], 0
    while i + 4 <= raw.size:
        wgs, pts, n_layer, batch = (int(x) for x in raw[i:i + 4])
        n = wgs * pts
        out.append((raw[i + 4:i + 4 + n].reshape(wgs, pts).astype(np.int64), n_layer, batch))
        i += 4 + n
    return out


def summarize_wide(trace, n_layer):
    """Median over workgroups of each interval, averaged over layers 1 .. L-1 (us per layer),
    the lm_head's intervals (us), the median layer time and the step span (first point of any
    workgroup to the last token pick)."""
    per = len(WIDE_POINTS)
    t = trace
    res = {"layer": {}, "lm_head": {}}
    for k, (name, _) in enumerate(WIDE_POINTS):
        acc = []
        for l in range(1, n_layer):
            cur = t[:, per * l + k]
            prev = t[:, per * l + k - 1] if k else t[:, per * (l - 1) + per - 1]
            acc.append(float(np.median(cur - prev)) * TICK_US)
        res["layer"][name] = float(np.mean(acc)) if acc else 0.0
    prev = t[:, per * (n_layer - 1) + per - 1]
    for k, (name, _) in enumerate(WIDE_LM):
        cur = t[:, per * n_layer + k]
        res["lm_head"][name] = float(np.median(cur - prev)) * TICK_US
        prev = cur
    if n_layer > 2:
        res["layer_us"] = float(np.median(t[:, per * (n_layer - 1)] - t[:, per])) * TICK_US / (n_layer - 2)
    res["step_us"] = float(t[:, per * n_layer + len(WIDE_LM) - 1].max() - t[:, 0].min()) * TICK_US
    return res


# The relay decode kernel (decode_relay.h, RelayArgs::trace): with FMLH_RELAY_TRACE=<file> set
# when an engine is created, every relay launch appends a header {steps, roles, points, n_layer,
# nq, n_head, nf, nf2, nA, nlm} and the device wall clock (100 MHz ticks) [step][role][point] of
# its first `steps` decode steps.  Roles of layer l: nq Q, nA n_head attention, nf FC and nf2
# row-sum workgroups, in that order; then the nlm lm_head roles.  Points of a role in a step
# (its item of sequence 0): 0 item start, 1 inputs settled, 2 mid-item, 3 outputs emitted, 4 the
# FC role's rows of x_{l+1} emitted (when it adds them up itself), 5 end of the role's last item
# of the step, 6 / 7 ticks spent waiting for inputs / working, summed over the step's items.
RELAY_CHAIN = [
    ("x_to_A", "x_l complete to the last attention role with its inputs (batch 1: x_l itself; "
               "else q / k_new / v_new from the Q team)"),
    ("A", "attention roles, inputs settled to dx1 emitted (the last of them)"),
    ("A_to_F", "last dx1 emitted to the last FC role with x_l and every dx1"),
    ("F", "FC roles, inputs settled to partials emitted (the last of them)"),
    ("F_to_rows", "last partial emitted to the last row of x_{l+1} emitted"),
]


def read_relay(path):
    """Relay launches in the file: a list of (array [steps][roles][points] of ticks, meta)."""
    raw = np.fromfile(path, dtype=np.uint64)
    out, i = [], 0
    while i + 10 <= raw.size:
        steps, roles, pts, n_layer, nq, n_head, nf, nf2, n_a, nlm = (int(x) for x in raw[i:i + 10])
        n = steps * roles * pts
        meta = dict(n_layer=n_layer, nq=nq, n_head=n_head, nf=nf, nf2=nf2, nA=n_a, nlm=nlm)
        out.append((raw[i + 10:i + 10 + n].reshape(steps, roles, pts).astype(np.int64), meta))
        i += 10 + n
    return out


def summarize_relay(trace, meta, steps=(1, 2, 3)):
    """Sequence 0's path through each layer (RELAY_CHAIN: the critical member of each team, us,
    averaged over layers 1 .. L-1), each team's waiting and working time per step (us, mean over
    its workgroups and the layers), and the step time (end of the lm_head role's last item),
    averaged over `steps`."""
    L, nq, H, nf, nf2 = (meta[k] for k in ("n_layer", "nq", "n_head", "nf", "nf2"))
    n_a, nlm = meta["nA"], meta["nlm"]
    per = nq + n_a * H + nf + nf2
    chain = {name: [] for name, _ in RELAY_CHAIN}
    chain["layer"] = []
    teams = {}
    step_us = []
    for s in steps:
        t = trace[s]
        team = {}
        for l in range(L):
            o = l * per
            team[l] = {"Q": t[o:o + nq], "A": t[o + nq:o + nq + n_a * H],
                       "F": t[o + nq + n_a * H:o + nq + n_a * H + nf],
                       "F2": t[o + nq + n_a * H + nf:o + per]}
            for k, v in team[l].items():
                if len(v):
                    teams.setdefault(k, []).append((float(v[:, 6].mean()) * TICK_US, float(v[:, 7].mean()) * TICK_US))

        def rows_out(l):
            return team[l]["F2"][:, 3].max() if nf2 else team[l]["F"][:, 4].max()

        for l in range(1, L):
            a, f = team[l]["A"], team[l]["F"]
            x_ready = rows_out(l - 1)
            chain["x_to_A"].append(a[:, 1].max() - x_ready)
            chain["A"].append(a[:, 3].max() - a[:, 1].max())
            chain["A_to_F"].append(f[:, 1].max() - a[:, 3].max())
            chain["F"].append(f[:, 3].max() - f[:, 1].max())
            chain["F_to_rows"].append(rows_out(l) - f[:, 3].max())
            chain["layer"].append(rows_out(l) - x_ready)
        lm = t[L * per:L * per + nlm]
        teams.setdefault("lm", []).append((float(lm[:, 6].mean()) * TICK_US, float(lm[:, 7].mean()) * TICK_US))
        step_us.append(float(lm[:, 5].max() - trace[s - 1][L * per:L * per + nlm, 5].max()) * TICK_US)
    res = {"chain": {k: float(np.mean(v)) * TICK_US for k, v in chain.items()},
           "teams": {k: {"wait": float(np.mean([w for w, _ in v])), "busy": float(np.mean([b for _, b in v]))}
                     for k, v in teams.items()},
           "step_us": float(np.mean(step_us)), "meta": meta}
    return res
