"""Writes the golden fixtures beside this file from the reference's own numpy modules.

    python tests/golden/make_golden.py [--reference /root/reference]

Imports the reference's numpy-only modules (``acrobot_np``, ``pendulum_aba_np``,
``hopper_np``, ``legged_np``; they import nothing but numpy and each other) and
samples exactly the functions whose float32 rounding sequence nothing else pins:

* ``acrobot_np._physics`` (acrobot_np.py:47-61): RK4 + wrap + clip, with numpy's own
  promotions inside ``_dsdt``/``_wrap``;
* ``pendulum_aba_np.aba_accelerations`` (pendulum_aba_np.py:30-99) at K = 1..64 and
  ``Pendulum._physics`` (pendulum_aba_np.py:118-125, RK4 dt 0.02);
* ``hopper_np.contact_impulse`` (hopper_np.py:80-109);
* ``legged_np.Legged._physics`` (legged_np.py:123-128) at C = 1, 2, 3, 4 and 4, 8, 16
  sweeps, eight chained steps, whose state the reference promotes to float64.

Inputs are drawn from seeded numpy generators; outputs are saved as plain arrays
(``.npz``, no pickles). Only the fixtures are committed and travel; the reference
code is read here and nowhere else.
"""

import argparse
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def acrobot(ref):
    import acrobot_np as A

    r = np.random.default_rng(101)
    n = 512
    state = np.stack([r.uniform(-np.pi, np.pi, n), r.uniform(-np.pi, np.pi, n),
                      r.uniform(-5 * np.pi, 5 * np.pi, n), r.uniform(-10 * np.pi, 10 * np.pi, n)]).astype(np.float32)
    state[:, :64] = r.uniform(-0.1, 0.1, size=(4, 64)).astype(np.float32)
    action = r.integers(0, 3, size=n).astype(np.int32)
    out = A._physics(state, action)
    np.savez_compressed(HERE / "acrobot_physics.npz", state=state, action=action, next_state=out)
    return {"acrobot_physics": (state.shape, out.dtype)}


def aba(ref):
    import pendulum_aba_np as P

    r = np.random.default_rng(202)
    arrays, info = {}, {}
    for k in (1, 2, 3, 4, 8, 16, 32, 64):
        n = 64
        th = r.uniform(-np.pi, np.pi, size=(k, n)).astype(np.float32)
        om = r.uniform(-3.0, 3.0, size=(k, n)).astype(np.float32)
        tq = r.uniform(-1.0, 1.0, size=n).astype(np.float32)
        acc = P.aba_accelerations(np, th, om, tq, k)
        arrays.update({f"k{k}_theta": th, f"k{k}_omega": om, f"k{k}_torque": tq, f"k{k}_acc": acc})
        info[f"aba k={k}"] = (th.shape, acc.dtype)
    for k in (2, 4, 16):
        n = 64
        state = np.concatenate([r.uniform(-0.5, 0.5, size=(k, n)), r.uniform(-1.0, 1.0, size=(k, n))]).astype(np.float32)
        action = r.integers(0, 3, size=n).astype(np.int32)
        out = P.Pendulum(k)._physics(state, action)
        arrays.update({f"rk4_k{k}_state": state, f"rk4_k{k}_action": action, f"rk4_k{k}_next": out})
        info[f"rk4 k={k}"] = (state.shape, out.dtype)
    np.savez_compressed(HERE / "pendulum_aba.npz", **arrays)
    return info


def contact(ref):
    import hopper_np as H

    r = np.random.default_rng(303)
    n = 4000
    Att = r.uniform(0.2, 3.0, n).astype(np.float32)
    Ann = r.uniform(0.2, 3.0, n).astype(np.float32)
    Atn = (r.uniform(-0.95, 0.95, n) * np.sqrt(Att * Ann)).astype(np.float32)
    wt = r.uniform(-2.0, 2.0, n).astype(np.float32)
    wn = r.uniform(-2.0, 1.0, n).astype(np.float32)
    depth = r.uniform(-0.02, 0.05, n).astype(np.float32)
    lt, ln = H.contact_impulse(np, Att, Atn, Ann, wt, wn, depth)
    np.savez_compressed(HERE / "contact_impulse.npz", Att=Att, Atn=Atn, Ann=Ann, wt=wt, wn=wn, depth=depth,
                        lt=np.asarray(lt), ln=np.asarray(ln))
    return {"contact_impulse": ((n,), np.asarray(lt).dtype)}


def legged(ref):
    import legged_np as L

    r = np.random.default_rng(404)
    arrays, info = {}, {}
    # the three-legged cases come last, so the earlier cases keep their draws
    cases = [(c, s, 0.0) for c in (1, 2, 4) for s in (4, 8, 16)] + [(4, 8, 20.0)] + [(3, s, 0.0) for s in (4, 8, 16)]
    for c, s, assist in cases:
        n, steps = 32, 8
        body = L.Legged(c, s)
        state = (body.stand[:, None] + r.uniform(-0.05, 0.05, size=(2 * (3 + c), n))).astype(np.float32)
        actions = r.integers(0, 3**c, size=(steps, n)).astype(np.int32)
        traj = [state]
        for t in range(steps):
            traj.append(body._physics(traj[-1], actions[t], assist))
        tag = f"c{c}_s{s}_a{int(assist)}"
        arrays[f"{tag}_state0"] = state
        arrays[f"{tag}_actions"] = actions
        arrays[f"{tag}_traj"] = np.stack([np.asarray(x, dtype=np.float64) for x in traj[1:]])
        arrays[f"{tag}_dtypes"] = np.array([str(np.asarray(x).dtype) for x in traj[1:]])
        info[f"legged {tag}"] = (state.shape, [str(np.asarray(x).dtype) for x in traj[1:3]])
    np.savez_compressed(HERE / "legged_physics.npz", **arrays)
    return info


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    for fn in (acrobot, aba, contact, legged):
        for k, v in fn(args.reference).items():
            print(k, v)


if __name__ == "__main__":
    main()
