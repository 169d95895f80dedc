"""Writes tests/golden/*.npz: small seeded inputs and the CPU oracle's outputs.

The reference ships no golden vectors (it has no tests), so these fixtures
freeze the oracle's results: tests/test_golden.py checks that the oracle still
reproduces them and that the HIP kernels match them. Regenerate only on a
deliberate change of the arithmetic contract:  python tests/golden/make_golden.py
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
import oracle  # noqa: E402

CASES = {
    # name: (T, H, block, tau, int8, sink_kv, sink_q)
    "b64_t200": (200, 1, 64, 0.9, False, (0, 0), (0, 0)),
    "b128_t300_sink": (300, 1, 128, 0.5, False, (0, 1), (0, 1)),
    "b64_t260_int8": (260, 1, 64, 0.8, True, (0, 0), (0, 0)),
}


def inputs(T, H, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((3, 1, T, H, 128)).astype(np.float32)
    x[1] += rng.standard_normal((1, 1, H, 128)).astype(np.float32) * 0.5  # key offset per head
    return [oracle.f32_to_bf16(t) for t in x]


def main():
    for seed, (name, (T, H, block, tau, int8, skv, sq)) in enumerate(CASES.items()):
        q, k, v = inputs(T, H, 100 + seed)
        p = oracle.prepare(q, k, v, block=block, tau=tau, int8=int8, sink_kv=skv, sink_q=sq)
        rows = [(0, h, i) for h in range(H) for i in range(p["NT"])]
        if int8:
            fwd = oracle.forward_int8_port(q, v, p, rows)
        else:
            fwd = oracle.forward_port(q, k, v, p, rows)
        out = np.concatenate([fwd[r] for r in rows]).reshape(H, -1, 128)[:, :T]
        NT = p["NT"]
        data = dict(q=q, k=k, v=v, T=T, H=H, block=block, tau=tau, int8=int8,
                    sink_kv=np.array(skv), sink_q=np.array(sq), kc=p["kc"][:, :NT], vc=p["vc"][:, :NT],
                    qbar=p["qbar"], kc_mean=p["kc_mean"], kc_var=p["kc_var"], thr=p["thr"],
                    counts=p["counts"], mask=p["mask"], out=out.astype(np.float16))
        if int8:
            data.update(qi=p["qi"], qs=p["qs"], ki=p["ki"], ks=p["ks"], vi=p["vi"],
                        vscale=p["vscale"])
        np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **data)
        print(name, "written")


if __name__ == "__main__":
    main()
