"""Phase timing of the fused verify run (diagnostic).

Builds the 35B-A3B-shaped synthetic model on the GPU, prefills the bench prompt, turns the fused
kernel's phase trace on, runs host-driven 2-lane verify steps and prints, per phase kind, the mean
time from the first workgroup to receive its inputs to the last workgroup done, the gap before it
(previous phase done to that first arrival), per workgroup the wait for inputs and the work after
them, the median sub-step marks, and the timeline of one DN and one attention layer. Times from the
device wall clock (100 MHz); "pass skew" is the time from the first to the last workgroup to receive
its inputs.

    python snapdragon-engine_amd/phase_trace.py [--prompt 512] [--steps 3]
"""
import argparse
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)

import oxe_amd as A  # noqa: E402

PHASES = {1: "proj", 2: "dn", 3: "scores", 4: "pv", 5: "out", 6: "router", 7: "experts", 8: "down", 9: "entry",
          10: "head"}
MARKS = {101: "experts: union", 102: "experts: gate/up loads issued", 103: "experts: issue drained",
         104: "experts: gate/up dot", 105: "experts: logits load", 106: "experts: route_wave",
         111: "proj: norm prologue", 113: "proj: int dots", 112: "proj: chains",
         117: "proj: int dots (again)", 118: "proj: chains (again)", 171: "out: int dots", 172: "out: chains", 121: "dn: conv", 122: "dn: norms + gates",
         123: "dn: delta rule", 124: "dn: head leader inputs", 125: "dn: head leader norm + store", 131: "router: norm prologue", 132: "router: f32 dots", 141: "pv: V tile to LDS",
         142: "pv: V.p + reduce", 143: "pv: scores load + max", 144: "pv: exp, sum, probabilities", 151: "scores: q/k prologue",
         161: "down: inputs", 162: "down: block dots", 163: "down: chains"}


def analyse(tr):
    """tr: [grid, events, 4] (id, start, passed, end). Returns (total_us, phase rows, mark rows)."""
    G = tr.shape[0]
    mains = []
    for g in range(G):
        ev = tr[g][(tr[g, :, 0] > 0) & (tr[g, :, 0] < 100)]
        mains.append(ev)
    n = min(len(m) for m in mains)
    mm = np.stack([m[:n] for m in mains]).astype(np.int64)
    ids = mm[0, :, 0]
    # a workgroup that takes no part in a phase records it with pass = 0: masked out below
    on = mm[:, :, 2] > 0
    start = np.ma.masked_array(mm[:, :, 1], ~on)
    pas = np.ma.masked_array(mm[:, :, 2], ~on)
    end = np.ma.masked_array(mm[:, :, 3], ~on)
    rel = pas.min(axis=0)
    done = end.max(axis=0)
    total = (done[-1] - start.min()) / 100.0
    agg = {}
    for k in range(n):
        name = PHASES.get(int(ids[k]), str(int(ids[k])))
        a = agg.setdefault(name, [0, 0.0, 0.0, 0.0])
        a[0] += 1
        a[1] += (done[k] - rel[k]) / 100.0
        a[2] += (rel[k] - done[k - 1]) / 100.0 if k > 0 else 0.0
        a[3] += (pas[:, k].max() - rel[k]) / 100.0
    marks = {}
    for g in range(G):
        ev = tr[g][tr[g, :, 0] >= 100].astype(np.int64)
        for e in ev:
            marks.setdefault(int(e[0]), []).append((e[3] - e[1]) / 100.0)
    # per workgroup: start -> inputs arrived ("wait") and inputs arrived -> end ("work")
    for k in range(n):
        name = PHASES.get(int(ids[k]), str(int(ids[k])))
        a = agg[name]
        if len(a) == 4:
            a += [[], []]
        a[4].append(np.ma.median(pas[:, k] - start[:, k]) / 100.0)
        a[5].append(np.ma.median(end[:, k] - pas[:, k]) / 100.0)
    return total, agg, marks, (ids, start, pas, end)


def phase_bytes(d, union, pos):
    """Algorithmic HBM bytes of one instance of each phase kind (Q8_0 rows: codes + fp16 scale per 32),
    for the run's two lanes at context position pos; union: routed experts per MoE layer (both lanes)."""
    q8 = lambda rows, k: rows * (k + k // 32 * 2)
    E, F, FF = d.n_embd, d.ff_exp, d.ff_shexp
    conv = d.ssm_d_inner + 2 * d.ssm_n_kheads * d.ssm_d_state        # q, k, v channels
    dn_rows = conv + d.ssm_d_inner + 2 * d.ssm_n_vheads               # [qkv; z; beta; alpha]
    at_rows = 2 * d.n_head * d.head_dim + 2 * d.n_head_kv * d.head_dim  # [q + gate; k; v]
    state = d.ssm_n_vheads * (d.ssm_d_inner // d.ssm_n_vheads) ** 2 * 4
    kv_row = d.n_head_kv * d.head_dim * 2
    return {
        "proj": (30 * q8(dn_rows, E) + 10 * q8(at_rows, E)) / 40.0,
        "dn": state * 3 + conv * 3 * 4 * 3 + conv * 4 * 4,
        "out": q8(E, d.ssm_d_inner),
        "router": d.n_expert * E * 4 + E * 4 + q8(2 * FF, E),
        "experts": union * q8(2 * F, E),
        "down": (union + 1) * q8(E, F),
        "scores": (pos + 2) * kv_row,
        "pv": (pos + 2) * kv_row,
        "head": q8(d.n_vocab, E),
    }


def timeline(ids, start, pas, end, k0, k1):
    """Rows (phase, start, pass, end) as min / median / max over workgroups, us from event k0's
    earliest start, for events [k0, k1)."""
    t0 = start[:, k0].min()
    rows = []
    for k in range(k0, k1):
        name = PHASES.get(int(ids[k]), str(int(ids[k])))
        q = [np.percentile((v[:, k].compressed() - t0) / 100.0, (0, 50, 100)) for v in (start, pas, end)]
        rows.append((name, q))
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--prompt", type=int, default=512)
    ap.add_argument("--steps", type=int, default=3)
    args = ap.parse_args()
    d = A.desc_35b_a3b()
    e = A.Engine(d, seed=0, n_ctx=args.prompt + 2 * args.steps + 256)
    if not e.fused:
        sys.exit("the fused run kernel is not available on this device")
    x = e.mtp_prefill(A.bench_prompt(args.prompt))
    e.set_trace(True)
    u0, c0 = e.counter(66), e.counter(67)
    for _ in range(args.steps):
        g = e.verify([x, (x + 1) % d.n_vocab])
        e.commit(1)
        x = int(g[0])
    union = (e.counter(66) - u0) / max(1, e.counter(67) - c0)
    total, agg, marks, ev = analyse(e.read_trace())
    pb = phase_bytes(d, union, e.pos)
    print(f"verify run (2 lanes, 40 layers + LM head) at position {e.pos}: {total:.1f} us; "
          f"routed experts per MoE layer (union of the lanes) {union:.2f}")
    print(f"{'phase':10s} {'count':>5s} {'release->done us':>17s} {'gap before us':>14s} {'pass skew us':>13s} "
          f"{'total us':>9s} {'wait med':>9s} {'work med':>9s} {'MB each':>8s} {'GB/s':>7s}")
    for name, (cnt, dur, gap, skew, wt, wk) in agg.items():
        mb = pb.get(name, 0.0) / 1e6
        gbs = mb * cnt / (dur + gap) * 1e3 if dur + gap > 0 else 0.0
        print(f"{name:10s} {cnt:5d} {dur / cnt:17.2f} {gap / cnt:14.2f} {skew / cnt:13.2f} {dur + gap:9.1f} "
              f"{np.mean(wt):9.2f} {np.mean(wk):9.2f} {mb:8.2f} {gbs:7.0f}")
    print("GB/s: the phase kind's algorithmic bytes over its total (release->done plus the gap before it)")
    ids = ev[0]
    # one DN layer and one attention layer in the middle of the run: start / inputs / end per phase
    for want in (2, 3):
        ks = [k for k in range(len(ids)) if ids[k] == want]
        if len(ks) < 2:
            continue
        k0 = ks[len(ks) // 2] - 1
        k1 = min(k0 + 7, len(ids))
        print(f"timeline of one {'DN' if want == 2 else 'attention'} layer (us; min / median / max over workgroups):")
        for name, q in timeline(*ev, k0, k1):
            print(f"  {name:8s} start {q[0][0]:6.2f} {q[0][1]:6.2f} {q[0][2]:6.2f} | inputs {q[1][0]:6.2f} {q[1][1]:6.2f} "
                  f"{q[1][2]:6.2f} | end {q[2][0]:6.2f} {q[2][1]:6.2f} {q[2][2]:6.2f}")
    print("sub-steps (median over workgroups and layers, us):")
    for i in sorted(marks):
        v = np.array(marks[i])
        print(f"  {MARKS.get(i, str(i)):32s} {np.median(v):6.2f}  (p90 {np.percentile(v, 90):.2f})")
    e.close()


if __name__ == "__main__":
    main()
