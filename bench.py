"""Benchmark of the fused attention hot path on one MI355X.

Workload (the configuration the headline metric is quoted on): bf16
fwd+bwd, B=8, H=16, L=4096, D=128, q/k/v/dO ~ N(0,1), key-padding keep-mask
[8,1,1,4096] whose per-batch valid length is drawn uniformly from
[1024, 4096], no bias, scale 1/sqrt(D).  One step = one forward + one
backward through the public drop-in (autograd over the C ABI), inputs
resident in HBM.

Counted FLOPs follow the flash-attention convention over *kept* (query, key)
pairs only: 4*D per pair forward (QK^T, PV) and 10*D backward, so 14*D per
pair per step.  ``value`` is counted TFLOP/s of the whole step.

``roofline`` is for the dominant kernel (the largest total time in the
timed step), timed live with HIP events recorded on the launch stream by the
library's profiling hook; its algorithmic FLOPs per launch are the GEMM work
that kernel does on kept pairs (dK/dV kernel: S, dP, dV, dK = 8*D per pair;
dQ kernel: S, dP, dQ = 6*D; forward: 4*D).

``cpu_baseline`` times the CPU oracle (numpy restatement of the reference's
attention, forward + closed-form backward, float32) on a bounded sample of
(batch, head) slices of the same workload on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

_ROOT = os.path.dirname(os.path.abspath(__file__))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0

B, H, L, D = 8, 16, 4096, 128
SEED = 2024


def _valid_lengths():
    rng = np.random.Generator(np.random.PCG64(SEED))
    return rng.integers(1024, L + 1, size=B)


def _cpu_baseline(valid, budget_s: float = 12.0):
    """Oracle fwd+bwd on (b, h) slices until ~budget_s of CPU time."""
    from oracle import attention as O

    try:
        from threadpoolctl import threadpool_info

        cores = max(
            (i.get('num_threads', 1) for i in threadpool_info()
             if i.get('user_api') == 'blas'),
            default=1,
        )
    except Exception:  # pragma: no cover
        cores = 1
    rng = np.random.Generator(np.random.PCG64(SEED + 1))
    scale = 1.0 / np.sqrt(D)
    flops = 0.0
    n = 0
    t0 = time.perf_counter()
    while True:
        b = n % B
        q = O.round_bf16(rng.standard_normal((1, 1, L, D), dtype=np.float32))
        k = O.round_bf16(rng.standard_normal((1, 1, L, D), dtype=np.float32))
        v = O.round_bf16(rng.standard_normal((1, 1, L, D), dtype=np.float32))
        g = O.round_bf16(rng.standard_normal((1, 1, L, D), dtype=np.float32))
        mask = (np.arange(L) < valid[b])[None, None, None, :]
        O.sdpa_forward(q, k, v, mask=mask, scale=scale)
        O.sdpa_backward(q, k, v, g, mask=mask, scale=scale)
        flops += 14.0 * D * L * float(valid[b])
        n += 1
        if time.perf_counter() - t0 >= budget_s:
            break
    dt = time.perf_counter() - t0
    return {
        'value': flops / dt / 1e12,
        'unit': 'TFLOP/s',
        'cores': int(cores),
        'kind': 'port',
        'sample': (
            f'{n} (b,h) slices of the workload (L={L}, D={D}, key-padding '
            f'mask of batch b), numpy oracle fwd+bwd in float32, {dt:.1f} s; '
            f'counted FLOPs as the GPU line'
        ),
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=5)
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument(
        '--copy-calibration',
        type=int,
        default=0,
        metavar='MIB',
        help='only run 5 device-to-device copies of MIB MiB (reference '
        'kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)',
    )
    args = ap.parse_args()
    world = int(os.environ.get('WORLD_SIZE', '1'))
    if args.gpus != 1 or world != 1:
        print(
            'bench.py measures one GPU only: every (batch, head) slab is '
            'independent, so the path shards over GPUs with no communication; '
            'no multi-GPU figure is produced by this build.',
            file=sys.stderr,
        )
        return 2

    import torch

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device='cuda:0').fill_(1)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({'copy_calibration_bytes_per_copy': n}), flush=True)
        return 0

    from nitrix_amd import _lib, scaled_dot_product_attention

    _lib.lib()
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    valid = _valid_lengths()
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32).to(
            torch.bfloat16
        )

    q = randn(B, H, L, D).requires_grad_()
    k = randn(B, H, L, D).requires_grad_()
    v = randn(B, H, L, D).requires_grad_()
    dout = randn(B, H, L, D)
    mask = (
        torch.arange(L, device=dev)[None, :]
        < torch.as_tensor(valid, device=dev)[:, None]
    )[:, None, None, :]
    kept_pairs = float(H * L * int(valid.sum()))
    step_flops = 14.0 * D * kept_pairs

    def step():
        q.grad = k.grad = v.grad = None
        out = scaled_dot_product_attention(q, k, v, mask=mask, backend='hip')
        out.backward(dout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    assert torch.isfinite(q.grad.float()).all(), 'non-finite gradient'

    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms = e0.elapsed_time(e1) / args.steps
    value = step_flops / (ms * 1e-3) / 1e12

    # Per-kernel durations (HIP events around each launch, same stream).
    prof_steps = max(3, min(args.steps, 10))
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(prof_steps):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kernels = {}
    for name in ('tilemap', 'fwd', 'delta', 'dkdv', 'dq'):
        tot, n = _lib.profile_read(name)
        if n:
            kernels[name] = {'avg_ms': tot / n, 'launches_per_step': n / prof_steps}
    _lib.profile_reset()
    per_pair = {'fwd': 4.0 * D, 'dkdv': 8.0 * D, 'dq': 6.0 * D}
    dom = max(
        (k_ for k_ in kernels if k_ in per_pair),
        key=lambda k_: kernels[k_]['avg_ms'] * kernels[k_]['launches_per_step'],
    )
    dom_flops = per_pair[dom] * kept_pairs
    achieved = dom_flops / (kernels[dom]['avg_ms'] * 1e-3) / 1e12
    fwd_tflops = 4.0 * D * kept_pairs / (kernels['fwd']['avg_ms'] * 1e-3) / 1e12

    cpu = None if args.no_cpu_baseline else _cpu_baseline(valid)

    line = {
        'metric': 'attention fwd+bwd TFLOP/s and % of bf16 MFMA peak at B8 H16 L4096 D128',
        'value': round(value, 3),
        'unit': 'TFLOP/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms, 4),
        'wall_s_timed': round(wall, 4),
        'pct_of_peak': round(100.0 * value / PEAK_BF16_TFLOPS, 3),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'bf16',
        'data': 'synthetic',
        'config': {
            'workload': 'bf16 attention fwd+bwd, key-padding mask (BASELINE configs[1])',
            'B': B,
            'H': H,
            'L': L,
            'D': D,
            'global_batch': B,
            'seq_len': L,
            'mask': f'key-padding [8,1,1,4096], valid lengths {valid.tolist()}',
            'bias': None,
            'causal': False,
            'counted_tflop_per_step': round(step_flops / 1e12, 4),
            'dense_equiv_tflop_per_step': round(14.0 * D * B * H * L * L / 1e12, 4),
            'parallelism': 'single GPU',
        },
        'fwd_tflops': round(fwd_tflops, 3),
        'fwd_pct_of_peak': round(100.0 * fwd_tflops / PEAK_BF16_TFLOPS, 3),
        'kernels': {k_: {kk: round(vv, 5) for kk, vv in v_.items()} for k_, v_ in kernels.items()},
        'roofline': {
            'kernel': dom,
            'bound': 'mfma',
            'achieved': round(achieved, 3),
            'peak': PEAK_BF16_TFLOPS,
            'unit': 'TFLOP/s',
            'frac': round(achieved / PEAK_BF16_TFLOPS, 4),
            'traffic': None,
        },
        'cpu_baseline': cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
