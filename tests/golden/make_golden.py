"""Write tests/golden/sample_small.json: the B=8, V=49152 fp32 N(0, 2^2) case.

Inputs are regenerated from the seed by loop-sglang_amd/workloads.py
(``sample_small``); only the outputs are stored.
  greedy_ids   torch.argmax(logits, -1) -- the reference's greedy call
               (python/loopsgl/model_executor/sample.py:110-111), run here on CPU.
  sampled_ids  T=0.7, top_k=50, top_p=0.9 with the seeded uniforms, from the CPU
               oracle (the reference's non-greedy path is flashinfer-python==0.6.6,
               CUDA-only and not installed, so no reference output exists for it).
  sampled_amb  the oracle's ambiguity flags for those rows.
Run:  python tests/golden/make_golden.py
"""
import json
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

import __graft_entry__  # noqa: E402
import oracle  # noqa: E402


def main():
    wl = __graft_entry__.package().workloads.sample_small("cpu", seed=0)
    x = wl["logits"]
    greedy = torch.argmax(x, dim=-1).to(torch.int32).tolist()
    ids, amb = oracle.sample(x.numpy(), wl["temperatures"].numpy(), wl["top_k"].numpy(),
                             wl["top_p"].numpy(), wl["uniforms"].numpy())
    out = dict(workload="sample_small", seed=0, B=8, V=49152, T=0.7, top_k=50, top_p=0.9,
               greedy_ids=greedy, sampled_ids=ids.tolist(), sampled_amb=amb.tolist(),
               logits_checksum=float(x.double().sum()))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sample_small.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print(path, out["greedy_ids"], out["sampled_ids"])


if __name__ == "__main__":
    main()
