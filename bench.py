"""Benchmark: batched hybrid key switching on one MI355X.

Workload (one "step"): 16 ciphertext polynomials d at 24 limbs of 50-bit primes, N = 2^16, each
key-switched with its own rotation key (rotations 1..16), dnum 3 (8-limb digits), 8 special
primes: ModUp -> key inner product -> ModDown, inputs and keys resident in HBM.

value = algorithmic bytes per step / step time, with the algorithmic bytes of the config:
per ciphertext d 12 MiB + key 96 MiB + (b, a) out 24 MiB = 138,412,032 B; 16 per step =
2,214,592,512 B.  The step time comes from HIP events on the stream the kernels run on.

cpu_baseline: this repository's CPU oracle (oracle/ckks_oracle.c, exact 128-bit integer
arithmetic, OpenMP over ciphertexts) runs the same 16 key switches once on the host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

BYTES_PER_CT = (12 + 96 + 24) * 2**20  # 138,412,032
CTS = 16
LIMBS = 24
HBM_PEAK_GBS = 8000.0
METRIC = "s per encrypted Llama-3-8B layer (128-tok prefill, 1 GPU); key-switch HBM GB/s"


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--seed", type=int, default=20261202)
    ap.add_argument("--chunk", type=int, default=CTS, help="ciphertexts per key-switch launch sequence")
    args = ap.parse_args()
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build has no multi-GPU path (each GPU box has one "
            "GPU); the key-switch batch would shard by ciphertext with zero exchange.",
            file=sys.stderr,
        )
        return 2

    import torch

    from holmes_amd import fhe

    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        return 1
    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, seed=args.seed)
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec)
    keys = []
    for r in range(1, CTS + 1):
        g = ctx.galois_element(r)
        ctx.rotation_keys[g] = client.rotation_key(g)
        keys.append(ctx.rotation_keys[g])
    rng = np.random.default_rng(args.seed)
    d_host = np.stack([np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(LIMBS)])
                       for _ in range(CTS)])
    d = torch.from_numpy(d_host).to(ctx.device)
    out_b = ctx.empty(CTS, LIMBS, ctx.N)
    out_a = ctx.empty(CTS, LIMBS, ctx.N)
    torch.cuda.synchronize()
    _log(f"setup {time.perf_counter() - t0:.1f}s (context, 16 keys of {keys[0].numel() * 8 / 2**20:.0f} MiB)")

    chunk = max(1, min(CTS, args.chunk))

    def step():
        for c0 in range(0, CTS, chunk):
            c1 = min(CTS, c0 + chunk)
            ctx.keyswitch(d[c0:c1], LIMBS, keys[c0:c1], out_b=out_b[c0:c1], out_a=out_a[c0:c1])

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms_events = ev0.elapsed_time(ev1) / args.steps
    ms_wall = wall * 1e3 / args.steps
    step_bytes = BYTES_PER_CT * CTS
    value = step_bytes / (ms_wall * 1e-3) / 1e9
    achieved = step_bytes / (ms_events * 1e-3) / 1e9
    _log(f"{args.steps} steps: {ms_wall:.3f} ms/step wall, {ms_events:.3f} ms/step events")

    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        threads = O.num_threads()
        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        keys_h = [k.cpu().numpy() for k in keys]
        _log(f"cpu baseline: 16 key switches on {threads} threads")
        c0 = time.perf_counter()
        wb, wa = orc.keyswitch_batch(LIMBS, d_host, keys_h)
        csec = time.perf_counter() - c0
        # the CPU result doubles as a parity spot check of the timed GPU output
        ok = bool(np.array_equal(out_b.cpu().numpy(), wb) and np.array_equal(out_a.cpu().numpy(), wa))
        cpu = {
            "value": round(step_bytes / csec / 1e9, 4),
            "unit": "GB/s",
            "cores": int(threads),
            "kind": "port",
            "sample": f"the full step (16 key switches, 24 limbs) once; {csec:.2f} s; "
                      f"bit-exact vs GPU: {ok}",
        }
        _log(f"cpu {csec:.2f}s, parity {ok}")

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": {
            "workload": "C2 batched hybrid key switch: 16 cts x 24 limbs, 16 distinct rotation keys",
            "N": ctx.N,
            "limbs": LIMBS,
            "prime_bits": 50,
            "dnum": 3,
            "special_primes": ctx.K,
            "batch": CTS,
            "algorithmic_bytes_per_step": step_bytes,
            "cts_per_launch": chunk,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "hck_keyswitch (whole ModUp -> inner product -> ModDown launch sequence per step)",
            "ms_per_launch": round(ms_events, 4),
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
