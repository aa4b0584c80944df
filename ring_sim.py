"""CPU simulation of the window kernel's K / V^T LDS ring schedule (correctness of slots)."""
def sim(T, R, loads_per_step_k=1, loads_per_step_v=1):
    # events: list of (step, kind) ; writes: slot -> list of (issue_step, tile)
    wk = {i: [] for i in range(R)}   # K slot writes
    wv = {i: [] for i in range(R)}
    ZERO = -1
    # prologue = step "-1": issues K(min(j,T-1)) into slot j for j<R, V(min(j,T-1)) into slot j for j<R-2, zero V slot R-1
    for j in range(R): wk[j].append((-1, min(j, T - 1)))
    for j in range(R - 2): wv[j].append((-1, min(j, T - 1)))
    wv[R - 1].append((-1, ZERO))
    # prologue waits for all (landed before step 0)
    reads = []  # (step, kind, slot, expected_tile)
    reads.append((-0.5, 'K', 0, 0))  # S(0) after the prologue wait
    for t in range(T):
        # at top of step t: wait until outstanding loads from steps >= t-(R-2) allowed in flight
        # issue
        wk[t % R].append((t, min(t + R, T - 1)))
        wv[(t + R - 2) % R].append((t, min(t + R - 2, T - 1)))
        reads.append((t, 'K', (t + 1) % R, t + 1 if t + 1 < T else None))
        reads.append((t, 'V', (t + R - 1) % R, t - 1 if t >= 1 else ZERO))
    reads.append((T, 'V', (T - 1) % R, T - 1))  # final PV after full wait
    ok = True
    for step, kind, slot, want in reads:
        if want is None:
            continue
        writes = (wk if kind == 'K' else wv)[slot]
        # writes issued at or before this step (issue step <= step); the read happens after the issue in the same step
        prior = [w for w in writes if w[0] <= step]
        last = prior[-1]
        # landed: issue step <= step - (R-1), or the prologue (-1) for reads at step >= -0.5, or the final full wait
        landed = last[0] == -1 or last[0] <= step - (R - 1) or step == T
        if last[1] != want or not landed:
            ok = False
            print("FAIL T=%d R=%d read %s slot %d at step %s wants %s, last write %s landed=%s" % (T, R, kind, slot, step, want, last, landed))
            break
    return ok

allok = all(sim(T, R) for T in range(1, 41) for R in (2, 3, 4, 5, 6))
print("ring schedule ok" if allok else "ring schedule FAILED")
