"""Writes sample_vectors.npz: the reference's own sample() (tokenrush/sample.py:30-51), run with
torch on the CPU in this container, over the inputs of sample_cases.py. Needs /root/reference;
run once, by hand: `python tests/golden/make_sample_vectors.py`. Nothing here runs on the GPU box,
and no test imports this script: the tests read only the .npz it writes."""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
import sample_cases as sc  # noqa: E402

REF = "/root/reference"


def main():
    sys.dont_write_bytecode = True  # the reference tree is read-only: no __pycache__ there
    sys.path.insert(0, REF)
    from tokenrush.sample import SamplingParams, sample    # the reference's module (imports torch only)
    torch.set_num_threads(8)
    out = {}
    for name, _, rows, V, seed, draws in sc.GROUPS:
        bits, u = sc.group_inputs(name)
        logits = torch.from_numpy(sc.bits_to_f32(bits)).to(torch.bfloat16)
        toks = np.zeros((rows, len(sc.PARAMS), draws), np.int64)
        for pi, (T, top_p, top_k) in enumerate(sc.PARAMS):
            p = SamplingParams("cpu")
            p.set(temperature=T, top_p=top_p, top_k=top_k)
            for d in range(draws):
                toks[:, pi, d] = sample(logits, p, torch.from_numpy(u[:, pi, d].copy())).numpy()
        out[name + "_tokens"] = toks
        out[name + "_logits_sha256"] = np.array(sc.digest(bits))
        out[name + "_u_sha256"] = np.array(sc.digest(u))
        print(name, rows, V, toks.size, "draws")
    out["params"] = np.array(sc.PARAMS, np.float64)
    out["torch_version"] = np.array(torch.__version__)
    np.savez_compressed(os.path.join(HERE, "sample_vectors.npz"), **out)


if __name__ == "__main__":
    main()
