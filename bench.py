"""Benchmark on one MI355X.

Default (``--workload c2``, the headline line): batched hybrid key switching, with the steady
prefill layer's seconds and decrypted error (the metric's first half, as ``--workload layer``
measures it) in the line's ``layer`` object (``--no-layer`` skips it).

Workload (one "step"): 16 ciphertext polynomials d at 24 limbs of 50-bit primes, N = 2^16, each
key-switched with its own rotation key (rotations 1..16), dnum 3 (8-limb digits), 8 special
primes: ModUp -> key inner product -> ModDown, inputs and keys resident in HBM.

value = algorithmic bytes per step / step time, with the algorithmic bytes of the config:
per ciphertext d 12 MiB + key 96 MiB + (b, a) out 24 MiB = 138,412,032 B; 16 per step =
2,214,592,512 B.  The step time comes from HIP events on the stream the kernels run on.

cpu_baseline: this repository's CPU oracle (oracle/ckks_oracle.c, exact 128-bit integer
arithmetic, OpenMP over ciphertexts) runs the same 16 key switches once on the host.

``--workload c3``: one Llama-3-8B q_proj projection (4096 x 4096, Gaussian std 0.02 weights
right-multiplied by a seeded randomized Hadamard) applied by the BSGS diagonal method (baby step
16, 512 plaintext rows per chunk) to 128 tokens x 4096 features encrypted feature-major into 16
ciphertexts at 20 limbs, scale 2^40.  A step is one whole projection, pack + encode of every
diagonal included (the reference encodes per chunk per call,
llama3fhe/operators/linear/operator.py:296-312).  Its line reports seconds per projection.

``--workload kv``: 128 PairFold token writes (4 ciphertexts each, 12 limbs) appended into one
HBM-pooled page: each append is one fused launch of eight polynomial sums into a fresh slot.
``--workload wire``: 16 ciphertexts at 24 limbs packed into one device buffer in the wire layout,
copied to pinned host memory and unpacked again.

``--workload c4``: the encrypted Llama-3-8B MLP block at 128 tokens (RMSNorm, gate/up 4096 ->
14336, SiLU degree 63, down 14336 -> 4096, one two-pass bootstrap of the output ciphertexts), 24
limbs, scale 2^50; its line reports seconds per block and the decrypted error against the float64
oracle of the same arithmetic.

``--workload layer``: one encrypted Llama-3-8B prefill layer at 128 tokens (the metric's "s per
encrypted layer"), steady state as the reference times its layer 10: input refresh, RMSNorm1,
complex QKV projections, RoPE, causal Alg2 attention over 32 heads (series inputs refreshed), W_O,
residual, refresh, the SwiGLU MLP block at width 14336, residual; 38 limbs of 50-bit primes, dnum 5,
scale 2^50; its line reports seconds per layer (and the model's first layer beside it) and the
decrypted error against the float64 model of the same polynomials.

``--workload c2wide``: the C2 shape (16 ciphertexts, 16 distinct rotation keys) on the reference's
production chain (assets/feature_major.json: 38 Q limbs of 60/59-bit primes, dnum 5, 8 special
primes of 60 bits), at the full 38 limbs, on the 64-bit integer kernels of the wide-prime path.

``--workload bootstrap``: one full-slot bootstrap (N = 2^16, 24 x 50-bit primes, dnum 3, scale
2^50, sparse ternary secret h = 192, level budget (3, 3)) of a ciphertext at 3 limbs; its line
reports ms per bootstrap and the precision of the refreshed slots.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

BYTES_PER_CT = (12 + 96 + 24) * 2**20  # 138,412,032
# HBM bytes one C2 step actually moves (all five kernels) come from two rocprofv3 --pmc runs of
# this workload (FETCH_SIZE x 2.0, the factor the stream workload's known read calibrates, plus
# WRITE_SIZE x 1.0), recorded with the SHA-256 of the kernel sources they were measured on; the
# line reports them only while the sources still match.
C2_TRAFFIC_RECORD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "keyswitch_c2_traffic.json")
CTS = 16
LIMBS = 24
HBM_PEAK_GBS = 8000.0
# C3: 4096 plaintexts x 20 limbs + keys + inputs + outputs, the algorithmic figure of the config
C3_BYTES = 45_629_833_216
C3_LIMBS = 20
C3_DIM = 4096
C3_TOKENS = 128
METRIC = "s per encrypted Llama-3-8B layer (128-tok prefill, 1 GPU); key-switch HBM GB/s"


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--no-layer", action="store_true",
                    help="c2: skip the steady prefill layer measured beside the key switch (the metric's first half)")
    ap.add_argument("--seed", type=int, default=20261202)
    ap.add_argument("--chunk", type=int, default=CTS, help="ciphertexts per key-switch launch sequence")
    ap.add_argument("--conv-engine", choices=("mfma", "valu"), default="mfma",
                    help="c2 / c2wide ModUp / ModDown conversion sums: int8 matrix cores or the VALU (same results)")
    ap.add_argument("--chain", choices=("50", "reference"), default="50",
                    help="layer: the 38-limb chain on 50-bit primes (FP64 kernels) or the reference's own "
                         "60/59-bit primes (assets/feature_major.json; 64-bit integer kernels)")
    ap.add_argument("--strategy", choices=("normal", "ext_double_hoist"), default="ext_double_hoist",
                    help="c3 giant steps: Horner chain (normal) or double hoisting in the extended basis "
                         "(both are hoist strategies of the reference's LinearOperatorConfig)")
    ap.add_argument("--workload", choices=("c1", "c2", "c2wide", "c3", "c4", "c5", "layer", "mul", "bootstrap", "kv",
                                           "wire", "stream"),
                    default="c2",
                    help="c2: batched key switch (headline); c1: one rotation + rescale (latency); "
                         "c3: q_proj BSGS projection; c4: encrypted MLP block; mul: 16 ciphertext products with "
                         "relinearisation and rescale at 24 limbs; bootstrap: one full-slot bootstrap "
                         "at 24 limbs; kv: 128 token appends into an HBM-pooled KV page; wire: 16 "
                         "ciphertexts packed into one device buffer and round-tripped through pinned "
                         "host memory; stream: the "
                         "residue negation kernel over 16 x 24 limbs, a plain read-once/write-once "
                         "stream of known size (HBM ceiling and counter calibration)")
    ap.add_argument("--write-traffic-record", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="no GPU: sum the last C2 step's five key-switch dispatches in the counter CSVs of "
                         "two `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE` runs of `bench.py --steps 2 "
                         "--warmup 0 --no-cpu --no-layer` and write the traffic record for the current kernel sources")
    args = ap.parse_args()
    if args.write_traffic_record:
        return write_traffic_record(*args.write_traffic_record)
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
    if args.workload == "c3":
        return run_c3(args)
    if args.workload == "c1":
        return run_c1(args)
    if args.workload == "stream":
        return run_stream(args)
    if args.workload == "mul":
        return run_mul(args)
    if args.workload == "bootstrap":
        return run_bootstrap(args)
    if args.workload == "c5":
        return run_c5(args)
    if args.workload == "layer":
        return run_layer(args)
    if args.workload == "c2wide":
        return run_c2wide(args)
    if args.workload == "c4":
        return run_c4(args)
    if args.workload == "kv":
        return run_kv(args)
    if args.workload == "wire":
        return run_wire(args)
    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, seed=args.seed)
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec)
    ctx.set_conversion_engine(args.conv_engine)
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
    traffic, traffic_rec = c2_traffic()
    if traffic is None:
        _log("roofline.traffic: no PMC record for these kernel sources (null)" if traffic_rec is None else
             "roofline.traffic: the PMC record was measured on other kernel sources (null)")

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
            "conv_engine": args.conv_engine,
            "traffic_record": None if traffic is None else {k: traffic_rec[k] for k in ("fetch_kib", "write_kib",
                                                                                       "fetch_scale", "measured")},
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "hck_keyswitch (whole ModUp -> inner product -> ModDown launch sequence per step)",
            "ms_per_launch": round(ms_events, 4),
        },
        "cpu_baseline": _cpu_annotated(cpu),
    }
    if not args.no_layer:
        # the metric's first half beside the key-switch half, measured in the same run
        del d, out_b, out_a, keys
        ctx.rotation_keys.clear()
        torch.cuda.empty_cache()
        line["layer"] = c2_layer_figures()
    print(json.dumps(line), flush=True)
    return 0


def run_c2wide(args) -> int:
    """C2 on the wide-prime path: 16 polynomials d at 38 limbs (q_0 60-bit, the rest 59-bit), each
    key-switched with its own rotation key (dnum 5: 5 digits of 8 limbs, 8 special 60-bit primes).
    Algorithmic bytes per ciphertext: d 38 limbs + key 2 x 5 x 46 limbs + (b, a) 2 x 38 limbs =
    574 limbs of 512 KiB."""

    import torch

    from holmes_amd import fhe

    ell = 38
    spec = fhe.CKKSContextSpec(depth=ell - 1, dnum=5, dcrt_bits=59, first_mod=60, scale_bits=59, seed=args.seed)
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec)
    ctx.set_conversion_engine(args.conv_engine)
    keys = []
    for r in range(1, CTS + 1):
        g = ctx.galois_element(r)
        ctx.rotation_keys[g] = client.rotation_key(g)
        keys.append(ctx.rotation_keys[g])
    rng = np.random.default_rng(args.seed)
    d_host = np.stack([np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(ell)])
                       for _ in range(CTS)])
    d = torch.from_numpy(d_host).to(ctx.device)
    out_b, out_a = ctx.empty(CTS, ell, ctx.N), ctx.empty(CTS, ell, ctx.N)
    torch.cuda.synchronize()
    _log(f"c2wide setup {time.perf_counter() - t0:.1f}s (38 limbs, 16 keys of {keys[0].numel() * 8 / 2**20:.0f} MiB)")

    def step():
        ctx.keyswitch(d, ell, keys, out_b=out_b, out_a=out_a)

    for _ in range(args.warmup):
        step()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_wall = (time.perf_counter() - w0) * 1e3 / args.steps
    ms_events = ev0.elapsed_time(ev1) / args.steps
    beta = -(-ell // ctx.alpha)
    step_bytes = CTS * (ell + 2 * beta * (ell + ctx.K) + 2 * ell) * ctx.N * 8
    _log(f"c2wide: {ms_wall:.3f} ms/step wall, {ms_events:.3f} ms/step events")
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        threads = O.num_threads()
        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        keys_h = [k.cpu().numpy() for k in keys]
        c0 = time.perf_counter()
        wb, wa = orc.keyswitch_batch(ell, d_host, keys_h)
        csec = time.perf_counter() - c0
        ok = bool(np.array_equal(out_b.cpu().numpy(), wb) and np.array_equal(out_a.cpu().numpy(), wa))
        cpu = {"value": round(step_bytes / csec / 1e9, 4), "unit": "GB/s", "cores": int(threads), "kind": "port",
               "sample": f"the full step (16 key switches, 38 limbs) once; {csec:.2f} s; bit-exact vs GPU: {ok}"}
        _log(f"cpu {csec:.2f}s, parity {ok}")
    achieved = step_bytes / (ms_events * 1e-3) / 1e9
    print(json.dumps({
        "metric": "key-switch HBM GB/s on the reference's production chain (38 limbs, 60/59-bit primes, dnum 5)",
        "value": round(step_bytes / (ms_wall * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_wall, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u64", "data": "synthetic",
        "config": {"workload": "C2 shape on the wide-prime path: 16 cts x 38 limbs, 16 distinct rotation keys",
                   "N": ctx.N, "limbs": ell, "prime_bits": [60, 59], "dnum": 5, "special_primes": ctx.K,
                   "batch": CTS, "algorithmic_bytes_per_step": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "hck_keyswitch on the wide path (whole launch sequence per step)",
                     "ms_per_launch": round(ms_events, 4)},
        "cpu_baseline": _cpu_annotated(cpu)}), flush=True)
    return 0


C1_BYTES = 149_946_368  # ct(24) in + KSK(24) + ct(23) out


def run_c1(args) -> int:
    """One rotation by 5^1 of one ciphertext at 24 limbs (fused automorphism + key switch), then
    rescale to 23 limbs, as one hck_rotate_rescale call (the ModDown and the rescale share one
    conversion pass): the latency case, with the oracle's result as the parity check.  ``two_step_ms``
    times hck_rotate followed by hck_rescale."""

    import torch

    from holmes_amd import fhe

    seed = 20261201
    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, seed=seed)
    client, ctx = fhe.generate_client_context(spec)
    g = ctx.galois_element(1)
    key = client.rotation_key(g)
    rng = np.random.default_rng(seed)
    c = [np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(LIMBS)])[None]
         for _ in range(2)]
    c0, c1 = (torch.from_numpy(x).to(ctx.device) for x in c)
    r0 = ctx.empty(2, LIMBS - 1, ctx.N)
    both = ctx.empty(2, LIMBS, ctx.N)

    def two_step():
        ctx.rotate_raw(c0, c1, LIMBS, g, key, out0=both[0:1], out1=both[1:2])
        ctx.rescale_raw(both, LIMBS, out=r0)

    for _ in range(args.warmup):
        two_step()
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    for _ in range(args.steps):
        two_step()
    torch.cuda.synchronize()
    ms_two = (time.perf_counter() - w0) * 1e3 / args.steps
    two = r0.clone()
    res = [None]

    def step():
        res[0] = ctx.rotate_rescale_raw(c0, c1, LIMBS, g, key)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_wall = (time.perf_counter() - w0) * 1e3 / args.steps
    ms = ev0.elapsed_time(ev1) / args.steps
    got = torch.stack([res[0][0][0], res[0][1][0]])
    if not torch.equal(got, two):
        raise RuntimeError("hck_rotate_rescale differs from hck_rotate + hck_rescale")
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        ok_key = orc.make_ksk(*client.key_inputs(g))
        t = time.perf_counter()
        w0_, w1_ = orc.rotate(LIMBS, g, c[0][0], c[1][0], ok_key)
        want = np.stack([orc.rescale(LIMBS, w0_), orc.rescale(LIMBS, w1_)])
        csec = time.perf_counter() - t
        ok = bool(np.array_equal(got.cpu().numpy(), want))
        cpu = {"value": round(csec * 1e3, 3), "unit": "ms", "cores": int(O.num_threads()), "kind": "port",
               "sample": f"the whole unit (rotation + rescale of both components) once; bit-exact vs GPU: {ok}"}
    achieved = C1_BYTES / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "ms per rotation + rescale (C1: 1 ct x 24 limbs)", "value": round(ms_wall, 4), "unit": "ms",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_wall, 4),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "u64", "data": "synthetic",
        "config": {"workload": "C1 single rotation by 5^1 + rescale, 24 -> 23 limbs, dnum 3, K 8",
                   "algorithmic_bytes_per_step": C1_BYTES, "two_step_ms": round(ms_two, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "rotation with the rescale fused into its ModDown (5 kernels)",
                     "ms_per_launch": round(ms, 4)},
        "cpu_baseline": _cpu_annotated(cpu)}), flush=True)
    return 0


# mul: 16 pairs at 24 limbs -> 16 products at 23 limbs; per pair a, b (2 x 24 MiB) + out (23 MiB),
# plus the one relinearisation key (96 MiB) every pair shares.
MUL_PAIRS = 16
MUL_BYTES = MUL_PAIRS * (24 + 24 + 23) * 2**20 + 96 * 2**20  # 1,291,845,632


def run_mul(args) -> int:
    """16 ciphertext x ciphertext products at 24 limbs: tensor product, relinearisation (key
    switch of the degree-2 term with the shared s^2 -> s key, added to the degree-0/1 terms), and
    rescale to 23 limbs -- the batched fhe.homo_mul_relin_rescale (hck_mul_relin_rescale: the
    ModDown and the rescale share one conversion pass).  The oracle's composition of the same
    operations on one pair is the parity check and the CPU sample."""

    import torch

    from holmes_amd import fhe

    seed = 20261213
    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, seed=seed)
    client, ctx = fhe.generate_client_context(spec)
    rng = np.random.default_rng(seed)
    host = [np.stack([np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(LIMBS)])
                      for _ in range(MUL_PAIRS)]) for _ in range(4)]
    a0, a1, b0, b1 = (torch.from_numpy(x).to(ctx.device) for x in host)
    res = [None]

    def step():
        res[0] = ctx.mul_relin_rescale_raw(a0, a1, b0, b1, LIMBS, ctx.relin_key, stacked=True)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        step()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_wall = (time.perf_counter() - w0) * 1e3 / args.steps
    ms = ev0.elapsed_time(ev1) / args.steps
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        rlk = orc.make_ksk(*client.relin_key_inputs())
        t = time.perf_counter()
        w0_, w1_ = orc.mul_relin(LIMBS, host[0][0], host[1][0], host[2][0], host[3][0], rlk)
        want = np.stack([orc.rescale(LIMBS, w0_), orc.rescale(LIMBS, w1_)])
        csec = time.perf_counter() - t
        got = res[0].cpu().numpy()
        ok = bool(np.array_equal(got[0][0], want[0]) and np.array_equal(got[1][0], want[1]))
        cpu = {"value": round(MUL_BYTES / (csec * MUL_PAIRS) / 1e9, 4), "unit": "GB/s",
               "cores": int(O.num_threads()), "kind": "port",
               "sample": f"one pair (product, relinearisation, rescale of both components) in {csec:.3f} s, "
                         f"x {MUL_PAIRS} pairs; bit-exact vs GPU: {ok}"}
    value = MUL_BYTES / (ms_wall * 1e-3) / 1e9
    achieved = MUL_BYTES / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "ciphertext products with relinearisation + rescale (16 pairs x 24 limbs), algorithmic GB/s",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_wall, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u64", "data": "synthetic",
        "config": {"workload": "16 ciphertext products at 24 limbs: tensor, relinearisation, rescale to 23",
                   "algorithmic_bytes_per_step": MUL_BYTES},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "tensor + 5 key-switch kernels, the rescale fused into the ModDown",
                     "ms_per_launch": round(ms, 4)},
        "cpu_baseline": _cpu_annotated(cpu)}), flush=True)
    return 0


# bootstrap / c4: the bytes of one unit are the HBM floors of the library calls it makes, summed
# from the call log of one run (limb = N x 8 bytes): key switch per item d + add + out (b, a) +
# its key 2 beta (limbs + K); product with relinearisation 4 in + 2 out per item + the shared key;
# MAC babies + plaintext rows + partial sums; rescale / ModRaise / weighted sums / linear
# combinations / elementwise ops and automorphisms their inputs and outputs.
class _Shape:
    __slots__ = ("shape",)

    def __init__(self, shape):
        self.shape = shape


class _CallLog:
    NAMES = ("keyswitch", "rotate_raw", "mul_relin_raw", "mul_relin_rescale_raw", "mul_relin_rescale_postop_raw",
             "relinearize_raw", "bsgs_mac",
             "rescale_raw", "modraise", "weighted_sum", "poly_op", "automorphism", "lincomb", "lincomb_rescale",
             "rotate_ext", "rotate_ext_sum", "hoist_digits", "rotate_hoisted", "rotate_rescale_raw", "moddown")

    def __init__(self, ctx):
        self.ctx = ctx
        self.calls = []

    @classmethod
    def _light(cls, v):
        """Shapes instead of tensors (the log must not keep a run's intermediates alive)."""

        if hasattr(v, "shape") and hasattr(v, "dtype"):
            return _Shape(tuple(v.shape))
        if isinstance(v, (list, tuple)):
            return [cls._light(x) for x in v]
        return v

    def __enter__(self):
        for name in self.NAMES:
            orig = getattr(self.ctx, name)

            def wrap(*a, _orig=orig, _name=name, **k):
                self.calls.append((_name, [self._light(x) for x in a], {kk: self._light(vv) for kk, vv in k.items()}))
                return _orig(*a, **k)

            setattr(self.ctx, name, wrap)
        return self

    def __exit__(self, *exc):
        for name in self.NAMES:
            delattr(self.ctx, name)

    def limbs_bytes(self):
        """(algorithmic limbs moved, [(kind, items, limbs)] of the key switches)."""

        ctx = self.ctx
        K = ctx.K
        beta = lambda l: (l + ctx.alpha - 1) // ctx.alpha  # noqa: E731
        total = 0
        ks = []
        for name, a, k in self.calls:
            if name == "keyswitch":
                d, l = a[0], int(a[1])
                B = int(d.shape[0])
                total += B * (l * (3 + (k.get("add") is not None)) + 2 * beta(l) * (l + K))
                ks.append(("rotation", B, l))
            elif name == "rotate_raw":
                l, B = int(a[2]), int(a[0].shape[0])
                total += B * (l * (4 + 2 * (k.get("acc") is not None)) + 2 * beta(l) * (l + K))
                ks.append(("rotation", B, l))
            elif name == "mul_relin_raw":
                l, B = int(a[4]), int(a[0].shape[0])
                total += B * 6 * l + 2 * beta(l) * (l + K)
                ks.append(("product", B, l))
            elif name == "mul_relin_rescale_raw":
                l, B = int(a[4]), int(a[0].shape[0])
                total += B * (4 * l + 2 * (l - 1)) + 2 * beta(l) * (l + K)
                ks.append(("product", B, l))
            elif name == "mul_relin_rescale_postop_raw":  # + the subtrahend when given
                l, B = int(a[4]), int(a[0].shape[0])
                total += B * (4 * l + 2 * (l - 1) * (1 + (k.get("sub") is not None))) + 2 * beta(l) * (l + K)
                ks.append(("product", B, l))
            elif name == "hoist_digits":  # c1 in, the extended digits out
                l, B = int(a[1]), int(a[0].shape[0])
                total += B * (l + beta(l) * (l + K))
            elif name == "rotate_hoisted":  # per item: c0, the input's digits, its key, the output
                l, items = int(a[2]), len(a[4])
                total += items * (3 * l + 3 * beta(l) * (l + K))
                ks.append(("rotation", items, l))
            elif name == "rotate_ext_sum":  # per member and output: c0, c1, key; per output the ext result
                l, G, B = int(a[2]), int(a[0].shape[0]), int(a[0].shape[1])
                acc = k.get("acc") if len(a) < 8 else a[7]
                total += G * B * (2 * l + 2 * beta(l) * (l + K)) + B * 2 * (l + K) * (1 + (acc is not None))
                ks.append(("rotation", G * B, l))
            elif name == "relinearize_raw":
                l, B = int(a[3]), int(a[0].shape[0])
                total += B * 5 * l + 2 * beta(l) * (l + K)
                ks.append(("product", B, l))
            elif name == "bsgs_mac":
                b0, pts, l, G = a[0], a[2], int(a[3]), int(a[4])
                ni = int(b0[0].shape[0])
                total += len(b0) * ni * 2 * l + int(pts.shape[0]) * l + 2 * G * ni * l
            elif name == "rescale_raw":
                x, l = a[0], int(a[1])
                total += int(x.shape[0]) * (2 * l - 1)
            elif name == "modraise":
                total += int(a[0].shape[0]) * (1 + int(a[1]))
            elif name == "weighted_sum":
                x, w, l = a[0], a[1], int(a[2])
                total += (int(x.shape[0]) + int(w.shape[0])) * l
            elif name == "poly_op":
                out, l = a[1], len(k["prime_idx"])
                total += int(out.shape[0]) * l * (3 if len(a) > 3 and a[3] is not None else 2)
            elif name == "automorphism":
                total += int(a[0].shape[0]) * 2 * int(a[2])
            elif name == "rotate_ext":
                l, B = int(a[2]), int(a[0].shape[0])
                total += B * (2 * l + 2 * (l + K) * (1 + (k.get("acc") is not None)) + 2 * beta(l) * (l + K))
                ks.append(("rotation", B, l))
            elif name == "moddown":
                l = int(a[1])
                total += int(a[0].shape[0]) * (2 * l + K)
            elif name == "lincomb":
                xs, l, outs = a[0], int(a[1]), a[2]
                total += (sum(len(r) for r in xs) + len(outs)) * l
            elif name == "lincomb_rescale":  # the terms in, the rescaled sums out
                xs, l, outs = a[0], int(a[1]), a[2]
                total += sum(len(r) for r in xs) * l + len(outs) * (l - 1)
            elif name == "rotate_rescale_raw":
                l, B = int(a[2]), int(a[0].shape[0])
                total += B * (2 * l + 2 * (l - 1) + 2 * beta(l) * (l + K))
                ks.append(("rotation", B, l))
        return total, ks


def run_bootstrap(args) -> int:
    """Full-slot bootstrap of one ciphertext at 3 limbs (holmes_amd.bootstrap, the
    easyfhe.bs.openfhe surface): ModRaise, CoeffToSlot (3 merged BSGS stages), EvalMod (degree-48
    Chebyshev + 3 double angles on the real and imaginary parts), SlotToCoeff (3 stages).
    ``graph_replay_ms`` times the same bootstrap replayed as one HIP graph (``RefreshGraph``)."""

    import math

    import torch

    from holmes_amd import bootstrap as B
    from holmes_amd import fhe

    seed = 20261230
    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, scale_bits=50,
                               secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=seed)
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec)
    bspec = B.BootstrapSpec(log_slots=ctx.logN - 1, level_budget=(3, 3))
    req = B.requirements(bspec, ctx.logN)
    client.generate_rotation_keys(req.rotations)
    prog = B.generate(ctx, bspec)
    rng = np.random.default_rng(seed)
    v = (rng.uniform(-1, 1, ctx.max_slots) + 1j * rng.uniform(-1, 1, ctx.max_slots)) / math.sqrt(2)
    ct = client.encrypt(v, cur_limbs=3)
    _log(f"context, {len(req.rotations)} keys, program: {time.perf_counter() - t0:.1f} s")
    out = B.bootstrap(ct, ctx, prog)  # encodes and caches the stage diagonals
    with _CallLog(ctx) as log:
        out = B.bootstrap(ct, ctx, prog)
    limbs_moved, ks = log.limbs_bytes()
    bs_bytes = limbs_moved * ctx.N * 8
    for _ in range(args.warmup):
        out = B.bootstrap(ct, ctx, prog)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(args.steps):
        out = B.bootstrap(ct, ctx, prog)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_wall = (time.perf_counter() - w0) * 1e3 / args.steps
    ms = ev0.elapsed_time(ev1) / args.steps
    err = float(np.max(np.abs(client.decrypt(out) - v)))
    # the same bootstrap replayed as one HIP graph (RefreshGraph), reported beside the eager value
    graph = B.RefreshGraph(ctx, prog, ct, iterations=1)
    for _ in range(args.warmup):
        gout = graph(ct)
    torch.cuda.synchronize()
    g0 = time.perf_counter()
    for _ in range(args.steps):
        gout = graph(ct)
    torch.cuda.synchronize()
    ms_graph = (time.perf_counter() - g0) * 1e3 / args.steps
    if any(not torch.equal(a, b) for a, b in zip(gout.cv, out.cv)):
        raise RuntimeError("the graph replay differs from the eager bootstrap")
    ks_items = sum(b for _, b, _ in ks)
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        g = ctx.galois_element(1)
        okey = orc.make_ksk(*client.key_inputs(g))
        rlk = orc.make_ksk(*client.relin_key_inputs())
        x = [np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(LIMBS)])
             for _ in range(4)]
        t = time.perf_counter()
        orc.rotate(LIMBS, g, x[0], x[1], okey)
        t_rot = time.perf_counter() - t
        t = time.perf_counter()
        orc.mul_relin(21, x[0][:21], x[1][:21], x[2][:21], x[3][:21], rlk)
        t_mul = time.perf_counter() - t
        total = sum(b * (t_rot * l / LIMBS if kind == "rotation" else t_mul * l / 21) for kind, b, l in ks)
        cpu = {"value": round(total * 1e3, 1), "unit": "ms", "cores": int(O.num_threads()), "kind": "port",
               "sample": f"extrapolated from the key switches alone: one rotation at 24 limbs ({t_rot:.3f} s) "
                         f"and one product + relinearisation at 21 limbs ({t_mul:.3f} s), scaled by limbs, "
                         f"over the {ks_items} key-switched items of one bootstrap"}
    achieved = bs_bytes / (ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "ms per full-slot CKKS bootstrap (N=2^16, 24 x 50-bit limbs, dnum 3)", "value": round(ms_wall, 3),
        "unit": "ms", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_wall, 3),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "u64", "data": "synthetic",
        "config": {"workload": "bootstrap of 1 ct at 3 limbs -> %d limbs; level budget (3, 3), EvalMod deg %d + "
                               "%d double angles, message ratio 2^-%d, sparse ternary h=192"
                               % (prog.output_limbs, bspec.cheb_degree, bspec.double_angle, bspec.message_ratio_bits),
                   "max_error_bits": round(-math.log2(err), 2), "key_switched_items": ks_items,
                   "algorithmic_bytes_per_step": bs_bytes, "graph_replay_ms": round(ms_graph, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole bootstrap (key switches, MACs, rescales, elementwise)", "ms_per_launch": round(ms, 3)},
        "cpu_baseline": _cpu_annotated(cpu)}), flush=True)
    return 0


KV_LIMBS = 12
KV_TOKENS = 128


def run_kv(args) -> int:
    """A step = 128 token writes appended into one page of an HBM-pooled PairFold layer cache
    (holmes_amd.kv_pages): the first opens the page by move, the others are fused four-ciphertext
    sums into a fresh pool slot.  Algorithmic bytes per fused append: the tail page and the token
    read, the new page written (3 x 8 polys x 12 limbs x 512 KiB)."""

    import torch

    from holmes_amd import backend, fhe
    from holmes_amd.context import Cipher, CipherState
    from holmes_amd.kv_pages import KVPagePool, PairFoldLayerCache, PairFoldTokenWrite

    seed = 20261241
    spec = fhe.CKKSContextSpec(depth=KV_LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, seed=seed)
    client, ctx = fhe.generate_client_context(spec)
    session = backend.EasyFHEContext(tensor=torch, fhe=fhe, client=client, context=ctx, max_slots=ctx.max_slots)
    rng = np.random.default_rng(seed)
    st = CipherState(cur_limbs=KV_LIMBS, scale_degree=1, scaling_factor=2.0**40)
    hi = np.array(ctx.primes[:KV_LIMBS], dtype=np.uint64)[None, None, :, None]
    src = torch.from_numpy(rng.integers(0, hi, (4, 2, KV_LIMBS, ctx.N), dtype=np.uint64)).cuda()
    pool = KVPagePool(ctx, KV_LIMBS, capacity=4)

    def tokens():
        # distinct handles per token (views of one resident source: the inputs are in HBM)
        return [PairFoldTokenWrite([Cipher([src[h, 0][None], src[h, 1][None]], st, slots=ctx.max_slots)
                                    for h in (0, 1)],
                                   [Cipher([src[h, 0][None], src[h, 1][None]], st, slots=ctx.max_slots)
                                    for h in (2, 3)], t) for t in range(KV_TOKENS)]

    def step(toks):
        cache = PairFoldLayerCache(pool=pool)
        for t in toks:
            cache.append(t, crypto_context=session)
        return cache

    for _ in range(args.warmup):
        step(tokens()).release()
    torch.cuda.synchronize()
    batches = [tokens() for _ in range(args.steps)]
    stream = torch.cuda.current_stream()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    ev0.record(stream)
    caches = []
    for b in batches:
        c = step(b)
        caches.append(c)
        c.release()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_wall = (time.perf_counter() - w0) * 1e3 / args.steps
    ms = ev0.elapsed_time(ev1) / args.steps
    # parity: the page of the last step is 128 x the source, modulo each prime
    q = hi.astype(object)
    c = step(tokens())
    got = np.stack([np.stack([h.cv[k][0].cpu().numpy() for k in range(2)]) for h in c.pages[0].handles])
    want = (src.cpu().numpy().astype(object) * KV_TOKENS % q).astype(np.uint64)
    ok = bool(np.array_equal(got, want))
    c.release()
    per_append = 3 * 8 * KV_LIMBS * ctx.N * 8
    step_bytes = (KV_TOKENS - 1) * per_append
    # the fused append kernel alone: the same launch (tail slot + token -> fresh slot), back to back
    xs = [[pool.buf[0, h, c, 0], src[h, c]] for h in range(4) for c in range(2)]
    outs = [pool.buf[1, h, c, 0] for h in range(4) for c in range(2)]
    ctx.lincomb(xs, KV_LIMBS, outs)
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(KV_TOKENS - 1):
        ctx.lincomb(xs, KV_LIMBS, outs)
    ev1.record(stream)
    torch.cuda.synchronize()
    k_ms = ev0.elapsed_time(ev1) / (KV_TOKENS - 1)
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        x = src.cpu().numpy()
        ones = np.ones((1, 2, KV_LIMBS), dtype=np.uint64)
        t = time.perf_counter()
        for h in range(4):
            for k in range(2):
                orc.weighted_sum(KV_LIMBS, np.stack([x[h, k], x[h, k]]), ones)
        csec = time.perf_counter() - t
        cpu = {"value": round(per_append / csec / 1e9, 3), "unit": "GB/s", "cores": int(O.num_threads()),
               "kind": "port", "sample": f"one append's eight sums with the oracle's weighted sum ({csec * 1e3:.1f} ms)"}
    achieved = per_append / (k_ms * 1e-3) / 1e9
    print(json.dumps({
        "metric": "PairFold KV page appends (HBM pool, 12 limbs), algorithmic GB/s", "value": round(
            step_bytes / (ms_wall * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_wall, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u64", "data": "synthetic",
        "config": {"workload": "128 token writes (4 cts x 12 limbs) into one pooled page; 127 fused appends",
                   "us_per_append": round(ms * 1e3 / (KV_TOKENS - 1), 2), "algorithmic_bytes_per_step": step_bytes,
                   "page_exact": ok, "note": "value includes the host-side ownership bookkeeping of each append; "
                                             "roofline is the fused append kernel alone"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "k_lincomb (8 groups x 2 terms per append)", "ms_per_launch": round(k_ms, 5)},
        "cpu_baseline": _cpu_annotated(cpu)}), flush=True)
    return 0


def run_wire(args) -> int:
    """A step = 16 ciphertexts at 24 limbs packed into one device buffer (wire layout), copied to
    pinned host memory and back, and unpacked: the bytes of the 16 ciphertexts cross HBM (gather),
    PCIe twice and HBM again (unpack)."""

    import torch

    from holmes_amd import fhe, wire
    from holmes_amd.context import Cipher, CipherState

    seed = 20261242
    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, seed=seed)
    client, ctx = fhe.generate_client_context(spec)
    rng = np.random.default_rng(seed)
    st = CipherState(cur_limbs=LIMBS, scale_degree=1, scaling_factor=2.0**40)
    hi = np.array(ctx.primes[:LIMBS], dtype=np.uint64)[None, :, None]
    cts = [Cipher([torch.from_numpy(rng.integers(0, hi, (1, LIMBS, ctx.N), dtype=np.uint64)).cuda() for _ in range(2)],
                  st, slots=ctx.max_slots) for _ in range(CTS)]
    buf = wire.device_pack(cts, primes=ctx.q_primes)
    nbytes = int(buf.numel())
    pinned = torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)
    back = torch.empty_like(buf)
    stream = torch.cuda.current_stream()

    def step():
        wire.device_pack(cts, primes=ctx.q_primes, out=buf)
        pinned.copy_(buf, non_blocking=True)
        back.copy_(pinned, non_blocking=True)
        return wire.device_unpack(back, count=CTS)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_pack = t_d2h = 0.0
    for _ in range(args.steps):
        torch.cuda.synchronize()
        a = time.perf_counter()
        wire.device_pack(cts, primes=ctx.q_primes, out=buf)
        torch.cuda.synchronize()
        b = time.perf_counter()
        pinned.copy_(buf, non_blocking=True)
        torch.cuda.synchronize()
        t_pack += (b - a) * 1e3
        t_d2h += (time.perf_counter() - b) * 1e3
    w0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    ms_wall = (time.perf_counter() - w0) * 1e3 / args.steps
    ok = all(torch.equal(a, b) for x, y in zip(out, cts) for a, b in zip(x.cv, y.cv))
    host = pinned.numpy().tobytes()
    t = time.perf_counter()
    serial = [wire.serialize(c, primes=ctx.q_primes) for c in cts[:4]]
    t_ser = (time.perf_counter() - t) / 4
    t = time.perf_counter()
    for s_ in serial:
        wire.deserialize(s_, device="cpu", primes=ctx.q_primes)
    t_de = (time.perf_counter() - t) / 4
    ct_bytes = 2 * LIMBS * ctx.N * 8
    pack_gbs = 2 * nbytes / (t_pack / args.steps * 1e-3) / 1e9
    print(json.dumps({
        "metric": "ciphertext wire round trip (16 cts x 24 limbs: pack, D2H + H2D pinned, unpack), GB/s of ciphertext",
        "value": round(nbytes / (ms_wall * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_wall, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u64", "data": "synthetic",
        "config": {"workload": "16 ciphertexts at 24 limbs through the wire layout", "bytes": nbytes,
                   "device_pack_ms": round(t_pack / args.steps, 4), "d2h_pinned_GBs": round(
                       nbytes / (t_d2h / args.steps * 1e-3) / 1e9, 2), "round_trip_exact": ok,
                   "host_serialize_GBs": round(ct_bytes / t_ser / 1e9, 3),
                   "host_deserialize_GBs": round(ct_bytes / t_de / 1e9, 3), "pinned_bytes": len(host)},
        "roofline": {"bound": "hbm", "achieved": round(pack_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(pack_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "device_pack (headers + one strided copy per component, host time included)",
                     "ms_per_launch": round(t_pack / args.steps, 4)},
        "cpu_baseline": None}), flush=True)
    return 0


def run_c4(args) -> int:
    """C4: one encrypted MLP block (holmes_amd.mlp.FeatureMajorMLPBlock) on 128 tokens x 4096
    features (16 ciphertexts); weights N(0, 0.02^2) rotated as a converted checkpoint's are (gate /
    up by a seeded randomized Hadamard on the 4096 axis, down by H_28 (x) H_512 on the 14336 axis,
    holmes_amd.hadamard.rotate_mlp_weights), gamma = 1 + N(0, 0.1^2), x ~ N(0, 1)."""

    import math

    import torch

    from holmes_amd import bootstrap as bs
    from holmes_amd import fhe, mlp
    from holmes_amd.hadamard import rotate_mlp_weights
    from holmes_amd.layouts import FeatureMajorPrefillLayout
    from holmes_amd.linear import LinearOperatorConfig

    seed = 20261204
    steps = int(args.steps) if args.steps != 20 else 1
    warmup = int(args.warmup) if args.warmup != 3 else 1
    t0 = time.perf_counter()
    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, scale_bits=50,
                               secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=seed)
    client, ctx = fhe.generate_client_context(spec)
    mspec = mlp.MLPBlockSpec()
    layout = FeatureMajorPrefillLayout()
    cfg = mlp.default_config()
    bspec = bs.BootstrapSpec(log_slots=15, level_budget=(3, 3))
    rots = set(mlp.FeatureMajorMLPBlock.rotations(mspec, layout, cfg)) | set(bs.requirements(bspec, 16).rotations)
    client.generate_rotation_keys(sorted(rots))
    prog = bs.generate(ctx, bspec)
    rng = np.random.default_rng(seed)
    D, Iw = mspec.hidden_dim, mspec.intermediate_width
    gate, up, down = rotate_mlp_weights(rng.normal(scale=0.02, size=(Iw, D)), rng.normal(scale=0.02, size=(Iw, D)),
                                        rng.normal(scale=0.02, size=(D, Iw)), seed + 1)
    gamma = 1.0 + 0.1 * rng.normal(size=D)
    block = mlp.FeatureMajorMLPBlock(ctx, gate, up, down, norm_weight=gamma, spec=mspec, layout=layout, config=cfg,
                                     bootstrap_program=prog)
    x = rng.normal(size=(128, D))
    cts = [client.encrypt(row, cur_limbs=ctx.L) for row in layout.pack(x)]
    _log(f"c4 setup {time.perf_counter() - t0:.1f} s: {len(rots)} rotation keys, {mspec.pages} feature pages")
    for _ in range(warmup):
        block.forward(cts)
    with _CallLog(ctx) as log:
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        out, stages = block.forward(cts)
        torch.cuda.synchronize()
        s_logged = time.perf_counter() - w0
    limbs_moved, ks = log.limbs_bytes()
    block_bytes = limbs_moved * ctx.N * 8
    secs = []
    for _ in range(steps):
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        out, stages = block.forward(cts)
        torch.cuda.synchronize()
        secs.append(time.perf_counter() - w0)
    s_wall = float(np.median(secs)) if secs else s_logged
    want = layout.pack(mlp.mlp_block_numpy(x, gate, up, down, gamma, mspec))
    err = max(float(np.max(np.abs(client.decrypt(o).real - want[i]))) for i, o in enumerate(out))
    _log(f"c4: {s_wall:.3f} s per block, stages {stages}, decrypted max error {err:.3e}")
    ks_items = sum(b for _, b, _ in ks)
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        g = ctx.galois_element(1)
        okey = orc.make_ksk(*client.key_inputs(g))
        xr = [np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(16)]) for _ in range(2)]
        t = time.perf_counter()
        orc.rotate(16, g, xr[0], xr[1], okey)
        t_rot = time.perf_counter() - t
        total = sum(b * t_rot * l / 16 for _, b, l in ks)
        cpu = {"value": round(total, 1), "unit": "s", "cores": int(O.num_threads()), "kind": "port",
               "sample": f"extrapolated from the key switches alone: one rotation at 16 limbs ({t_rot:.3f} s), scaled "
                         f"by limbs, over the {ks_items} key-switched items of one block (MACs, encodes, "
                         f"rescales not counted)"}
    achieved = block_bytes / s_wall / 1e9
    print(json.dumps({
        "metric": "s per encrypted Llama-3-8B MLP block (C4: 128 tokens, 4096 -> 14336 -> 4096, one bootstrap)",
        "value": round(s_wall, 4), "unit": "s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(s_wall * 1e3, 2), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "u64", "data": "synthetic",
        "config": {"workload": "C4 MLP block: RMSNorm (deg-15 rsqrt), gate/up 4 pages x 4096x4096 BSGS (baby 64), SiLU deg 63 "
                               "on [-16,16], down, two-pass bootstrap of 16 cts; 24 limbs, scale 2^50, dnum 3",
                   "decrypted_max_error": err, "error_bits": round(-math.log2(err), 2),
                   "stage_seconds": {k: round(v, 4) for k, v in stages.items()},
                   "key_switched_items": ks_items, "algorithmic_bytes_per_step": block_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole block (call-log algorithmic bytes: keys, diagonals, inputs/outputs of each call)",
                     "ms_per_launch": round(s_wall * 1e3, 2)},
        "cpu_baseline": _cpu_annotated(cpu)}), flush=True)
    return 0


def run_c5(args) -> int:
    """C5: one encrypted Llama-3-8B decode step, one layer (holmes_amd.decode.DecodeLayer): the
    token at position 256 against a 256-token encrypted KV cache in HBM-resident PairFold pages
    (K at 13 limbs, V at 7), GQA 32/8/128, RoPE theta 500000, Alg2 softmax (exp on [-4, 4] of
    s / (2 sqrt(d)), i.e. scores in [-8, 8], one 1/sqrt round), SwiGLU MLP 4096 -> 14336 -> 4096,
    five two-pass refreshes.  Weights N(0, 0.02^2), gammas 1 + N(0, 0.1^2), hidden and cached K/V
    N(0, 1).  Each timed step extends a fresh copy of the cache (the copy is not timed)."""

    import math
    import types

    import torch

    from holmes_amd import bootstrap as bs
    from holmes_amd import decode as Dm
    from holmes_amd import fhe

    seed = 20261205
    steps = int(args.steps) if args.steps != 20 else 3
    warmup = int(args.warmup) if args.warmup != 3 else 1
    t0 = time.perf_counter()
    cs = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, scale_bits=50,
                             secret_key_dist="SPARSE_TERNARY", hamming_weight=192, seed=seed)
    client, ctx = fhe.generate_client_context(cs)
    spec = Dm.DecodeSpec()
    history = 256
    pages = history // spec.page_size + 1
    rots = Dm.decode_key_rotations(pages)
    client.generate_rotation_keys(rots)
    progs = [bs.generate(ctx, b) for b in Dm.decode_bootstrap_specs()]
    ops = Dm.CipherOps(ctx, progs[0], progs[1])
    rng = np.random.default_rng(seed)
    w = Dm.random_weights(spec, rng)
    layer = Dm.DecodeLayer(ops, w, spec)
    x = rng.normal(size=spec.hidden_dim)
    ck = rng.normal(size=(history, 1024))
    cv = rng.normal(size=(history, 1024))
    S = float(ctx.scale_at(ctx.L))
    base = Dm.encrypt_kv_history(client, ck, cv, spec, S)
    xin = client.encrypt(Dm.lr8(x), cur_limbs=ctx.L)
    cc = types.SimpleNamespace(fhe=fhe, context=ctx)
    _log(f"c5 setup {time.perf_counter() - t0:.1f} s: {len(rots)} rotation keys")
    for _ in range(warmup):
        layer.forward(xin, base.clone(), position=history, crypto_context=cc)
    cache = base.clone()
    with _CallLog(ctx) as log:
        torch.cuda.synchronize()
        out, stages, _ = layer.forward(xin, cache, position=history, crypto_context=cc)
        torch.cuda.synchronize()
    limbs_moved, ks = log.limbs_bytes()
    step_bytes = limbs_moved * ctx.N * 8
    secs, all_stages = [], []
    for _ in range(steps):
        cache = base.clone()
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        out, stages, _ = layer.forward(xin, cache, position=history, crypto_context=cc)
        torch.cuda.synchronize()
        secs.append(time.perf_counter() - w0)
        all_stages.append(stages)
    s_wall = float(np.median(secs))
    stages = {k: float(np.median([st[k] for st in all_stages])) for k in all_stages[0]}
    ref = Dm.decode_layer_numpy(x, ck, cv, w, spec, position=history)
    got = client.decrypt(out)[::8].real
    err = float(np.max(np.abs(got - ref["output"])))
    mag = float(np.max(np.abs(ref["output"])))
    _log(f"c5: {s_wall:.3f} s per step, stages {stages}, decrypted max error {err:.3e} of magnitude {mag:.2f}, "
         f"softmax vs exact {ref['softmax_vs_exact']:.2e}, in range {ref['in_range']}")
    ks_items = sum(b for _, b, _ in ks)
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        g = ctx.galois_element(1)
        okey = orc.make_ksk(*client.key_inputs(g))
        xr = [np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(16)]) for _ in range(2)]
        t = time.perf_counter()
        orc.rotate(16, g, xr[0], xr[1], okey)
        t_rot = time.perf_counter() - t
        total = sum(b * t_rot * l / 16 for _, b, l in ks)
        cpu = {"value": round(total, 1), "unit": "s", "cores": int(O.num_threads()), "kind": "port",
               "sample": f"extrapolated from the key switches alone: one rotation at 16 limbs ({t_rot:.3f} s), scaled "
                         f"by limbs, over the {ks_items} key-switched items of one step (MACs, encodes, "
                         f"rescales not counted)"}
    achieved = step_bytes / s_wall / 1e9
    print(json.dumps({
        "metric": "s per encrypted Llama-3-8B decode step, one layer (C5: 256-token KV, 17-limb attention cap)",
        "value": round(s_wall, 4), "unit": "s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(s_wall * 1e3, 2), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "u64", "data": "synthetic",
        "config": {"workload": "C5 decode step: RMSNorm, complex QKV (512 diagonals), RoPE'd routes into PairFold pages, "
                               "QK over 3 pages, Alg2 softmax, PV, W_O (2x128 diagonals), SwiGLU 4096->14336->4096; "
                               "5 two-pass refreshes; 24 limbs, scale 2^50, dnum 3",
                   "decrypted_max_error": err, "output_magnitude": mag,
                   "error_bits_relative": round(-math.log2(err / mag), 2),
                   "softmax_vs_exact": ref["softmax_vs_exact"], "in_range": ref["in_range"],
                   "refreshes": ops.refreshes // max(1, steps + warmup + 1),
                   "stage_seconds": {k: round(v, 4) for k, v in stages.items()},
                   "key_switched_items": ks_items, "algorithmic_bytes_per_step": step_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole step (call-log algorithmic bytes: keys, diagonals, inputs/outputs of each call)",
                     "ms_per_launch": round(s_wall * 1e3, 2)},
        "cpu_baseline": _cpu_annotated(cpu)}), flush=True)
    return 0


def _cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo) and its logical CPU count."""

    name = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    name = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{name} ({os.cpu_count()} logical CPUs visible)"


def _cpu_annotated(cpu):
    """A cpu_baseline dict with the host CPU model added (None stays None)."""

    return None if cpu is None else {**cpu, "cpu_model": _cpu_model()}


# The sources the C2 step's kernels are built from: the FP64 key-switch kernels and their entry
# point, the tile layout, the arithmetic and the context tables they read.  The traffic record holds
# only while these match (a change to the wide-prime kernels does not move C2's bytes).
C2_KERNEL_SOURCES = ("context.hip", "internal.hpp", "keyswitch.hip", "ksfused.hip", "modarith.hpp", "tile_layout.hpp")


def kernel_sources_sha256() -> str:
    """SHA-256 over the C2 kernels' sources (name and bytes of each file of C2_KERNEL_SOURCES)."""

    import hashlib

    root = os.path.join(os.path.dirname(os.path.abspath(__file__)), "holmes_amd", "csrc")
    h = hashlib.sha256()
    for name in sorted(C2_KERNEL_SOURCES):
        h.update(name.encode())
        with open(os.path.join(root, name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def write_traffic_record(fetch_dir: str, write_dir: str) -> int:
    """The C2 traffic record from two PMC runs: per counter, the last five key-switch dispatches
    (one C2 step: INTT rows, ModUp, P-limb rows, ModDown, Q-limb rows) are summed (KiB); FETCH_SIZE
    is scaled by 2.0 and WRITE_SIZE by 1.0, the factors a plain stream kernel of known size reads
    (profiles/stream_calibration.md)."""

    import csv
    import datetime
    import glob

    def last_step_kib(d: str) -> float:
        per_dispatch: dict[int, float] = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f) as fh:
                for r in csv.DictReader(fh):
                    if "k_ks_" in r["Kernel_Name"]:
                        i = int(r["Dispatch_Id"])
                        per_dispatch[i] = per_dispatch.get(i, 0.0) + float(r["Counter_Value"])
        if len(per_dispatch) < 5:
            raise SystemExit(f"{d}: fewer than five key-switch dispatches in the counter CSVs")
        return sum(v for _, v in sorted(per_dispatch.items())[-5:])

    fetch, write = last_step_kib(fetch_dir), last_step_kib(write_dir)
    rec = {"sources_sha256": kernel_sources_sha256(), "fetch_kib": round(fetch, 1), "write_kib": round(write, 1),
           "fetch_scale": 2.0, "write_scale": 1.0, "traffic_bytes": int(round((2.0 * fetch + write) * 1024)),
           "measured": f"{datetime.date.today().isoformat()} rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on "
                       "bench.py --steps 2 --warmup 0 --no-cpu --no-layer"}
    with open(C2_TRAFFIC_RECORD, "w") as f:
        json.dump(rec, f, indent=1)
    print(json.dumps(rec))
    return 0


def c2_traffic():
    """(bytes per step, record) from the traffic record if it was measured on these sources."""

    try:
        with open(C2_TRAFFIC_RECORD) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None, None
    if rec.get("sources_sha256") != kernel_sources_sha256():
        return None, rec
    return int(rec["traffic_bytes"]), rec


def _layer_setup(seed: int = 20261206, chain: str = "50") -> dict:
    """The N1 workload: the 38-limb context (``chain``: 50-bit primes, or the reference's 60/59-bit
    ones with its refresh schedule, prefill.reference_chain_spec), every rotation key and refresh
    program of the layer, the first-layer and steady-state PrefillLayer objects, and the encrypted
    input (128 tokens x 4096 features N(0, 1), 16 ciphertexts) at the top of the chain and at the
    steady input level."""

    from holmes_amd import fhe
    from holmes_amd import prefill as P
    from holmes_amd.layouts import FeatureMajorPrefillLayout

    t0 = time.perf_counter()
    spec = P.PrefillSpec() if chain == "50" else P.reference_chain_spec()
    client, ctx = fhe.generate_client_context(P.prefill_context_spec(seed, chain=chain))
    rng = np.random.default_rng(seed)
    w = P.random_weights(spec, rng)
    first, rots = P.setup_prefill_layer(client, ctx, w, spec)
    steady = P.PrefillLayer(ctx, w, spec, program=first.program, config=first.config, steady=True,
                            programs=first.programs)
    layout = FeatureMajorPrefillLayout()
    x = rng.normal(size=(128, spec.hidden_dim))
    packed = layout.pack(x)
    cts_first = [client.encrypt(row, cur_limbs=ctx.L) for row in packed]
    cts_steady = [client.encrypt(row, cur_limbs=P.LAYER_OUTPUT_LIMBS) for row in packed]
    _log(f"layer setup {time.perf_counter() - t0:.1f} s: {len(rots)} rotation keys, {ctx.L} limbs, dnum {ctx.dnum}")
    return {"P": P, "ctx": ctx, "client": client, "rng": rng, "spec": spec, "w": w, "x": x, "layout": layout,
            "first": first, "steady": steady, "rots": rots, "cts_first": cts_first, "cts_steady": cts_steady}


def _time_layer(layer, cts, label: str, steps: int, warmup: int):
    """(last output, median seconds, median stage seconds) over ``steps`` forwards after ``warmup``."""

    import torch

    for _ in range(warmup):
        layer.forward(cts)
    secs, all_stages = [], []
    out = None
    for _ in range(steps):
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        out, stages = layer.forward(cts)
        torch.cuda.synchronize()
        secs.append(time.perf_counter() - w0)
        all_stages.append(stages)
        _log(f"{label} step {len(secs)}: {secs[-1]:.3f} s")
    med = float(np.median(secs))
    return out, med, {k: float(np.median([st[k] for st in all_stages])) for k in all_stages[0]}


def _layer_error(L: dict, out, ref=None):
    """(float64 model, max decrypted error over every slot, output magnitude) of a layer output."""

    P, client, layout = L["P"], L["client"], L["layout"]
    if ref is None:
        ref = P.prefill_layer_numpy(L["x"], L["w"], L["spec"])
    want = layout.pack(ref["output"])
    err = max(float(np.max(np.abs(client.decrypt(o).real - want[i]))) for i, o in enumerate(out))
    return ref, err, float(np.max(np.abs(ref["output"])))


def c2_layer_figures(steps: int = 2, warmup: int = 1) -> dict:
    """The metric's other half for the default line: the steady-state N1 layer's seconds (median of
    ``steps`` after ``warmup``) and its decrypted error against the float64 model."""

    import math

    L = _layer_setup()
    out, s_wall, stages = _time_layer(L["steady"], L["cts_steady"], "steady layer", steps, warmup)
    _, err, mag = _layer_error(L, out)
    _log(f"steady layer: {s_wall:.3f} s, error {err:.3e} (2^{math.log2(err):.2f}), magnitude {mag:.2f}")
    return {"metric": "s per encrypted Llama-3-8B layer (128-tok prefill, 1 GPU)",
            "value": round(s_wall, 4), "unit": "s", "steps": steps, "warmup": warmup,
            "workload": "N1 prefill layer, steady state (as --workload layer): 128 tokens, 38 limbs of 50-bit "
                        "primes, dnum 5, scale 2^50; input, residual and series inputs refreshed",
            "decrypted_max_error": err, "error_bits": round(-math.log2(err), 2), "output_magnitude": round(mag, 4),
            "stage_seconds": {k: round(v, 4) for k, v in stages.items()}}


def run_layer(args) -> int:
    """N1: one encrypted Llama-3-8B prefill layer (holmes_amd.prefill.PrefillLayer) on 128 tokens x
    4096 features (16 ciphertexts, 38-limb chain): weights N(0, 0.02^2), gammas 1 + N(0, 0.1^2),
    x ~ N(0, 1).  ``value`` is the steady-state layer, as the reference times its layer 10
    (bench/t2_layer.py): the input arrives at the previous layer's output level and is refreshed
    first, and the softmax's series inputs are refreshed (each refresh raised only as far as its
    consumer needs); the model's first layer (fresh
    input at 38 limbs, one refresh) is timed beside it.  Keys, the refresh program and the weight
    objects are built before the timed region; every weight diagonal is encoded inside it (per
    projection chunk, as the reference encodes per call), while the attention's slot constants keep
    their encodings across steps."""

    import math

    import torch

    steps = int(args.steps) if args.steps != 20 else 3
    warmup = int(args.warmup) if args.warmup != 3 else 1
    L = _layer_setup(chain=args.chain)
    P, ctx, client, rng = L["P"], L["ctx"], L["client"], L["rng"]
    first, steady, spec, w, x = L["first"], L["steady"], L["spec"], L["w"], L["x"]
    rots, cts_steady = L["rots"], L["cts_steady"]
    out_f, s_first, stages_f = _time_layer(first, L["cts_first"], "first layer", steps, warmup)
    out, s_wall, stages = _time_layer(steady, cts_steady, "steady layer", steps, warmup)
    with _CallLog(ctx) as log:
        torch.cuda.synchronize()
        steady.forward(cts_steady)
        torch.cuda.synchronize()
    limbs_moved, ks = log.limbs_bytes()
    layer_bytes = limbs_moved * ctx.N * 8
    ref, err, mag = _layer_error(L, out)
    _, err_f, _ = _layer_error(L, out_f, ref)
    _log(f"steady layer: {s_wall:.3f} s, stages {stages}, error {err:.3e}; first layer {s_first:.3f} s, "
         f"error {err_f:.3e}; magnitude {mag:.2f}")
    ks_items = sum(b for _, b, _ in ks)
    cpu = None
    if not args.no_cpu:
        from oracle import oracle as O

        orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
        g = ctx.galois_element(1)
        okey = orc.make_ksk(*client.key_inputs(g))
        xr = [np.stack([rng.integers(0, ctx.primes[i], ctx.N, dtype=np.uint64) for i in range(16)]) for _ in range(2)]
        t = time.perf_counter()
        orc.rotate(16, g, xr[0], xr[1], okey)
        t_rot = time.perf_counter() - t
        total = sum(b * t_rot * l / 16 for _, b, l in ks)
        cpu = {"value": round(total, 1), "unit": "s", "cores": int(O.num_threads()), "kind": "port",
               "sample": f"extrapolated from the key switches alone: one rotation at 16 limbs of the 38-limb chain "
                         f"({t_rot:.3f} s), scaled by limbs, over the {ks_items} key-switched items of one "
                         f"steady-state layer (MACs, encodes, rescales not counted)"}
    achieved = layer_bytes / s_wall / 1e9
    print(json.dumps({
        "metric": "s per encrypted Llama-3-8B layer (128-tok prefill, 1 GPU)",
        "value": round(s_wall, 4), "unit": "s", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": round(s_wall * 1e3, 2), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "u64", "data": "synthetic",
        "config": {"workload": "N1 prefill layer, steady state, 128 tokens: input refresh, RMSNorm1 (deg-15 rsqrt), "
                               "complex QKV (2 x 4096x4096 BSGS), RoPE, causal Alg2 attention 32/8/128 (exp deg 15 "
                               "and rsqrt deg 31 on refreshed inputs), W_O, residual, refresh, SwiGLU "
                               "4096->14336->4096 (SiLU deg 63), residual; refresh passes: input "
                               f"{spec.input_refresh_iterations}, exp input {spec.exp_refresh_iterations}, inverse "
                               f"square root input {spec.rsqrt_refresh_iterations}, residual "
                               f"{spec.residual_refresh_iterations}; 38 limbs of "
                               + ("50-bit primes, scale 2^50" if args.chain == "50" else
                                  "the reference's 60/59-bit primes, scale 2^59") + ", dnum 5",
                   "chain": args.chain,
                   "decrypted_max_error": err, "output_magnitude": mag, "error_bits": round(-math.log2(err), 2),
                   "softmax_vs_exact": ref["softmax_vs_exact"], "in_range": ref["in_range"],
                   "rotation_keys": len(rots), "refreshed_items_per_layer": steady.ops.refreshes // (warmup + steps + 1),
                   "stage_seconds": {k: round(v, 4) for k, v in stages.items()},
                   "first_layer_seconds": round(s_first, 4), "first_layer_error": err_f,
                   "first_layer_stage_seconds": {k: round(v, 4) for k, v in stages_f.items()},
                   "key_switched_items": ks_items, "algorithmic_bytes_per_step": layer_bytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "whole layer (call-log algorithmic bytes: keys, diagonals, inputs/outputs of each call)",
                     "ms_per_launch": round(s_wall * 1e3, 2)},
        "cpu_baseline": _cpu_annotated(cpu)}), flush=True)
    return 0


def run_stream(args) -> int:
    import torch

    from holmes_amd import _native as nat
    from holmes_amd import fhe

    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, seed=args.seed)
    ctx = fhe.CKKSContext(spec)
    idx = ctx.q_prime_idx(LIMBS)
    a = ctx.zeros(CTS, LIMBS, ctx.N)
    out = ctx.empty(CTS, LIMBS, ctx.N)
    nbytes = 2 * a.numel() * 8
    for _ in range(args.warmup):
        ctx.poly_op(nat.HCK_OP_NEG, out, a, prime_idx=idx)
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(args.steps):
        ctx.poly_op(nat.HCK_OP_NEG, out, a, prime_idx=idx)
    ev1.record(stream)
    torch.cuda.synchronize()
    ms = ev0.elapsed_time(ev1) / args.steps
    print(json.dumps({"workload": "stream: k_poly_op<NEG> over 16 x 24 limbs", "bytes_per_launch": nbytes,
                      "read_bytes": nbytes // 2, "write_bytes": nbytes // 2, "launches": args.steps,
                      "ms_per_launch": round(ms, 5), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 2)}), flush=True)
    return 0


def run_c3(args) -> int:
    import torch

    from holmes_amd import fhe, linear
    from holmes_amd.hadamard import randomized_hadamard_right
    from holmes_amd.layouts import FeatureMajorPrefillLayout

    seed = int(args.seed)
    steps = int(args.steps) if args.steps != 20 else 3
    warmup = int(args.warmup) if args.warmup != 3 else 1
    t0 = time.perf_counter()
    cfg = linear.LinearOperatorConfig(baby_steps=16, baby_anchor_step=-1, max_plaintext_rows=512,
                                      hoist_strategy=args.strategy)
    layout = FeatureMajorPrefillLayout(seq_len=C3_TOKENS, hidden_dim=C3_DIM, slots=32768)
    lanes = layout.tokens_per_cipher
    plan = cfg.plan(dimension=C3_DIM, token_lanes=lanes)
    spec = fhe.CKKSContextSpec(depth=LIMBS - 1, dnum=3, dcrt_bits=50, first_mod=50, seed=seed,
                               rotations=linear.bsgs_rotations(plan, args.strategy))
    client, ctx = fhe.generate_client_context(spec)
    rng = np.random.default_rng(seed)
    w = randomized_hadamard_right(rng.normal(scale=0.02, size=(C3_DIM, C3_DIM)), seed + 1)
    x = rng.normal(size=(C3_TOKENS, C3_DIM))
    packed = layout.pack(x)
    cts = [client.encrypt(packed[c], cur_limbs=C3_LIMBS, scaling_factor=2.0**40) for c in range(layout.cipher_count)]
    op = linear.LinearOperator(crypto_context=ctx, token_lanes=lanes, config=cfg)
    weight = linear.LinearWeight(w, crypto_context=ctx)
    torch.cuda.synchronize()
    _log(f"c3 setup {time.perf_counter() - t0:.1f}s: {len(spec.rotations)} keys, {len(cts)} cts at "
         f"{C3_LIMBS} limbs, {plan.plaintext_chunks} chunks x {plan.chunk_giants} giants x {plan.baby_steps} babies")

    outs = None
    for _ in range(warmup):
        outs = op.project(cts, weight)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    ev0.record(stream)
    for _ in range(steps):
        outs = op.project(cts, weight)
    ev1.record(stream)
    torch.cuda.synchronize()
    s_wall = (time.perf_counter() - w0) / steps
    s_events = ev0.elapsed_time(ev1) * 1e-3 / steps
    _log(f"{steps} projections: {s_wall:.4f} s wall, {s_events:.4f} s events")

    # decrypted spot check of two ciphertexts against float64 W' x
    want = layout.pack(x @ w.T)
    err = 0.0
    for c in (0, layout.cipher_count - 1):
        got = client.decrypt(outs[c]).real
        err = max(err, float(np.max(np.abs(got - want[c]))))
    _log(f"decrypted max abs error {err:.3e} (bound 2^-16 = {2.0**-16:.3e})")

    ks_per_projection = len(cts) * (plan.baby_rotation_count + sum(c.giant_count - 1 for c in plan.chunks)
                                    + sum(1 for c in plan.chunks if c.giant_base))
    cpu = None
    if not args.no_cpu:
        cpu = _c3_cpu_sample(ctx, client, plan, w, cts, ks_per_projection)

    achieved = C3_BYTES / s_events / 1e9
    line = {
        "metric": "s per q_proj projection (C3: 4096x4096 BSGS, 16 cts x 20 limbs)",
        "value": round(s_wall, 5),
        "unit": "s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(s_wall * 1e3, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": {
            "workload": "C3 q_proj BSGS: 4096x4096 Hadamard-rotated N(0, 0.02^2) weight, 128 tokens "
                        "feature-major in 16 cts x 20 limbs, baby 16, 512 plaintext rows per chunk",
            "N": ctx.N,
            "limbs": C3_LIMBS,
            "chunks": plan.plaintext_chunks,
            "key_switches": ks_per_projection,
            "hoist_strategy": args.strategy,
            "algorithmic_bytes_per_step": C3_BYTES,
            "decrypted_max_abs_error": err,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "whole projection (babies, pack + encode, MAC, Horner giant key switches, rescale)",
            "ms_per_launch": round(s_events * 1e3, 3),
        },
        "cpu_baseline": _cpu_annotated(cpu),
    }
    print(json.dumps(line), flush=True)
    return 0


def _c3_cpu_sample(ctx, client, plan, w, cts, ks_count):
    """Times the oracle on a bounded sample and extrapolates to one projection: one rotation at
    20 limbs (x key switches per projection), one chunk's MAC for one input (x chunks x inputs)
    and the encode of 8 diagonal rows (x 4096 / 8)."""

    from oracle import oracle as O

    threads = O.num_threads()
    orc = O.OracleContext(16, ctx.L, ctx.K, ctx.alpha, ctx.primes)
    g = ctx.galois_element(plan.giant_offset)
    key = orc.make_ksk(*client.key_inputs(g))
    c0 = cts[0].cv[0].cpu().numpy()[0, :C3_LIMBS]
    c1 = cts[0].cv[1].cpu().numpy()[0, :C3_LIMBS]
    t = time.perf_counter()
    orc.rotate(C3_LIMBS, g, c0, c1, key)
    t_ks = time.perf_counter() - t
    chunk = plan.chunks[0]
    scale = float(ctx.rescale_divisor_at(C3_LIMBS))
    rows = O.pack_diagonals(w, plan.token_lanes, 0, plan.baby_steps, chunk.giant_base, chunk.giant_count,
                            ctx.max_slots)
    idx = list(range(C3_LIMBS))
    t = time.perf_counter()
    enc = [orc.encode_real(rows[i], scale, idx)[0] for i in range(8)]
    t_enc8 = time.perf_counter() - t
    pts = np.stack(enc * (rows.shape[0] // 8))
    babies = np.stack([np.stack([c0, c1])] * plan.baby_steps)
    t = time.perf_counter()
    orc.bsgs_mac(C3_LIMBS, plan.baby_steps, chunk.giant_count, pts, babies)
    t_mac = time.perf_counter() - t
    total = ks_count * t_ks + plan.plaintext_chunks * len(cts) * t_mac + (C3_DIM // 8) * t_enc8
    _log(f"cpu sample: rotation {t_ks:.3f}s, chunk MAC {t_mac:.2f}s, 8 encodes {t_enc8:.3f}s -> "
         f"{total:.1f} s per projection")
    return {
        "value": round(total, 2),
        "unit": "s",
        "cores": int(threads),
        "kind": "port",
        "sample": f"extrapolated: 1 rotation at 20 limbs ({t_ks:.3f} s) x {ks_count}, one chunk MAC for "
                  f"one input ({t_mac:.2f} s) x {plan.plaintext_chunks * len(cts)}, 8 row encodes "
                  f"({t_enc8:.3f} s) x {C3_DIM // 8}",
    }


if __name__ == "__main__":
    sys.exit(main())
