"""Write the golden fixtures from the reference's own compiled attention.

Run in the build container (where /root/reference exists), after
`make -C oracle`:

    python tests/golden/gen_golden.py

For every case of cases.py it drives oracle/_ref/libjanas_ref_attn.so -
/root/reference/src/llm/attention.c built from its sources - through the
reference's API with FLOAT scores (the exact path; no calibration, nothing
written under ~/.cache), in calls of at most 64 tokens as the engine makes
them (model_attn.c:284-294), and stores the outputs with a digest of the
inputs in tests/golden/<case>.npz. Where the reference's INT16 scores apply
(an int8 cache, head size a multiple of 16) the same calls are made again
with INT16 asked for, into the key out_int16. It also checks on the way that
the block equals token-by-token calls bit for bit (attention.h:13-16), as
the reference's test does.
"""
import os
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

from cases import CASES, KV_I16, digest, int16_case, make_inputs  # noqa: E402

from oracle import orc  # noqa: E402

MAX_BLOCK = 64  # JANAS_ATTN_MAX_BLOCK, attention.h:26


def reference_outputs(name, inp, scores=1):
    c = CASES[name]
    ra = orc.RefAttention(c["n_head"], c["n_kv"], c["hd"], c["n_ctx"], 4,
                          scores)
    lib = ra.lib()
    try:
        if lib.janas_attn_scores_mode(ra.a) != scores:
            raise AssertionError(f"{name}: scores mode not taken")
        if c["kv"] == KV_I16:
            lib.janas_attn_set_kv16(ra.a, 1)
        if c.get("window"):
            lib.janas_attn_set_window(ra.a, c["window"])
        if c.get("ring"):
            lib.janas_attn_set_ring(ra.a, 1)
        if c.get("scale") is not None:
            lib.janas_attn_set_scale(ra.a, c["scale"])
        q, last = inp["q"], inp["last"]
        n, pos0 = c["n"], c["pos0"]
        k, v, ks, vs = inp["k"], inp["v"], inp["ks"], inp["vs"]
        out = np.zeros_like(q)
        for s in range(0, n, MAX_BLOCK):
            m = min(MAX_BLOCK, n - s)
            ls = None if last is None else last[s:s + m]
            out[s:s + m] = ra.run(np.ascontiguousarray(q[s:s + m]), k, ks, v,
                                  vs, pos0 + s, ls)
        if last is None:
            for j in range(n):
                one = ra.run(np.ascontiguousarray(q[j:j + 1]), k, ks, v, vs,
                             pos0 + j)
                if not np.array_equal(one.view(np.uint32),
                                      out[j:j + 1].view(np.uint32)):
                    raise AssertionError(f"{name}: block != token {j}")
        return out
    finally:
        ra.close()


def main():
    # the mode is asked for at create; the variable would override it
    os.environ.pop("JANAS_ATTN", None)
    os.environ["HOME"] = tempfile.mkdtemp()
    os.environ.pop("XDG_CACHE_HOME", None)
    for name in CASES:
        inp = make_inputs(name)
        out = reference_outputs(name, inp)
        extra = {}
        if int16_case(name):
            extra["out_int16"] = reference_outputs(name, inp, scores=2)
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, out=out, digest=np.array(digest(inp)),
                            **extra)
        print(f"{name}: {out.shape}{' +int16' if extra else ''} -> "
              f"{os.path.relpath(path, ROOT)}")


if __name__ == "__main__":
    main()
