"""Benchmark of the fused attention hot path on one MI355X.

Default workload (``--config c2``, the configuration the headline metric is
quoted on, BASELINE ``configs[1]``): bf16 fwd+bwd, B=8, H=16, L=4096, D=128,
q/k/v/dO ~ N(0,1), key-padding keep-mask [8,1,1,4096] whose per-batch valid
length is drawn uniformly from [1024, 4096], no bias, scale 1/sqrt(D).  One
step = one forward + one backward through the public drop-in (autograd over
the C ABI), inputs resident in HBM.

The other BASELINE configurations are available as ``--config c1|c3|c4|c5``
(one JSON line per run, same keys):

* ``c1`` fp32 fwd, B1 H4 L256 D64, full bias [1,4,256,256];
* ``c3`` bf16 causal fwd+bwd, B4 H32 L8192 D128;
* ``c4`` bf16 fwd, full per-head bias [2,16,8192,8192], q/k/v [2,16,8192,64]
  (HBM-bound: ``roofline`` is GB/s against 8 TB/s);
* ``c5`` bf16 fwd+bwd, B1 H8 L32768 D64, block-sparse keep-mask [1,1,L,L]
  from 128x128 blocks kept with p=0.25 (diagonal kept), bias [1,8,1,L]
  (with its gradient).

``--config ssm`` measures the sibling fused selective scan instead (fp32
fwd+bwd, batch 8, L 2048, d 1536, n 16), in (batch, step, channel) elements
per second, with its compulsory HBM bytes for the roofline.

Counted FLOPs follow the flash-attention convention over *kept* (query, key)
pairs only: 4*D per pair forward (QK^T, PV) and 10*D backward.  ``value`` is
counted TFLOP/s of the whole step.

``roofline`` is for the dominant kernel (the largest total time in the
step), timed live with HIP events recorded on the launch stream by the
library's profiling hook.  MFMA-bound kernels count the GEMM work they do on
kept pairs (dK/dV: S, dP, dV, dK = 8*D per pair; dQ: S, dP, dQ = 6*D;
forward: 4*D); the HBM-bound biased forward counts its compulsory bytes
(bias, q, k, v, o, lse once).

``cpu_baseline`` times the CPU oracle (numpy restatement of the reference's
attention, forward [+ closed-form backward], float32) on a bounded sample of
the same workload -- blocks of query rows of single (batch, head) slices --
and reports it in the same counted-FLOP unit.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

_ROOT = os.path.dirname(os.path.abspath(__file__))
if _ROOT not in sys.path:
    sys.path.insert(0, _ROOT)

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_F32_TFLOPS = 157.3  # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0

# HBM bytes per launch of each configuration's dominant kernel, measured with
# rocprofv3 FETCH_SIZE / WRITE_SIZE passes (scaled x2 / x1 by a copy-kernel
# calibration); the passes, the calibration and every kernel's figures are in
# profiles/attention_hbm_traffic_c1_c5.md.  Reported as roofline.traffic.
# TRAFFIC_SRC is the fingerprint (_src_fingerprint) of the attention kernel
# sources the passes ran; when the sources differ, the figure describes other
# kernels and is reported as stale (traffic null, the old figure beside it).
TRAFFIC_SRC = '31b32cd5e083de76'
MEASURED_TRAFFIC = {
    'c1': ('fwd', 6102721),
    'c2': ('dkdv', 910444756),
    'c3': ('dkdv', 1619918515),
    'c4': ('fwd', 4431184901),
    'c5': ('dkdv', 706542360),
}
# VALU instructions (wave64) of the selective scan's backward pass (all five
# kernels) per step at the ssm configuration, transcendental instructions
# weighted 4: the
# rocprofv3 SQ_INSTS_VALU / SQ_INSTS_VALU_TRANS_F32 counts of its kernels in
# profiles/selective_scan_valu_counters.md.
SSM_BWD_VALU_WAVE_INSTS = 2.5654e8
# Fingerprint of nxa_ssm.hip + nxa_common.h when the counts were taken.
SSM_VALU_SRC = 'fa3803c37f913189'
SSM_VALU_SOURCE = 'profiles/selective_scan_valu_counters.md (rocprofv3 SQ_INSTS_VALU, SQ_INSTS_VALU_TRANS_F32)'
PEAK_VALU_TLANEOPS = 256 * 4 * 32 * 2.4e9 / 1e12  # 78.6 T lane-instructions/s
TRAFFIC_SOURCE = 'profiles/attention_hbm_traffic_c1_c5.md (rocprofv3 FETCH_SIZE x2 + WRITE_SIZE x1)'
SEED = 2024

METRIC = 'attention fwd+bwd TFLOP/s and % of bf16 MFMA peak at B8 H16 L4096 D128'

CONFIGS = {
    'c1': dict(
        io='f32', B=1, H=4, L=256, D=64, bias='full', mask=None, causal=False,
        bwd=False,
        workload='fp32 attention fwd, full bias [1,4,256,256] (BASELINE configs[0])',
    ),
    'c2': dict(
        io='bf16', B=8, H=16, L=4096, D=128, bias=None, mask='keypad', causal=False,
        bwd=True,
        workload='bf16 attention fwd+bwd, key-padding mask (BASELINE configs[1])',
    ),
    'c3': dict(
        io='bf16', B=4, H=32, L=8192, D=128, bias=None, mask=None, causal=True,
        bwd=True,
        workload='bf16 causal attention fwd+bwd (BASELINE configs[2])',
    ),
    'c4': dict(
        io='bf16', B=2, H=16, L=8192, D=64, bias='full', mask=None, causal=False,
        bwd=False,
        workload='bf16 attention fwd, full per-head bias [2,16,8192,8192] (BASELINE configs[3])',
    ),
    'c5': dict(
        io='bf16', B=1, H=8, L=32768, D=64, bias='row', mask='blocksparse', causal=False,
        bwd=True,
        workload='bf16 attention fwd+bwd, block-sparse mask [1,1,L,L] (128x128 blocks, '
        'p=0.25, diagonal kept), bias [1,8,1,L] (BASELINE configs[4])',
    ),
    # Measurement lines of the widened path (not BASELINE configurations).
    'c2f16': dict(
        io='f16', B=8, H=16, L=4096, D=128, bias=None, mask='keypad', causal=False,
        bwd=True,
        workload='fp16 attention fwd+bwd, key-padding mask (C2 in fp16)',
    ),
    'c2qk': dict(
        io='bf16', B=8, H=16, L=4096, D=128, bias=None, mask='keypad', causal=False,
        bwd=True, qk_norm=True,
        workload='bf16 attention fwd+bwd with qk_norm, key-padding mask (C2 with qk-norm)',
    ),
    'c2qkf': dict(
        io='bf16', B=8, H=16, L=4096, D=128, bias=None, mask='keypad', causal=False,
        bwd=False, qk_norm=True,
        workload='bf16 attention fwd (no backward) with qk_norm, key-padding mask',
    ),
    'd64': dict(
        io='bf16', B=8, H=16, L=4096, D=64, bias=None, mask=None, causal=False,
        bwd=True,
        workload='bf16 attention fwd+bwd, head dim 64, no mask',
    ),
    'w256': dict(
        io='bf16', B=4, H=16, L=4096, D=256, bias=None, mask=None, causal=False,
        bwd=True,
        workload='bf16 attention fwd+bwd, head dim 256',
    ),
    'c2f32': dict(
        io='f32', B=8, H=16, L=4096, D=128, bias=None, mask='keypad', causal=False,
        bwd=True,
        workload='fp32 attention fwd+bwd, key-padding mask (C2 in fp32, the dtype of the '
        "reference's fused kernel)",
    ),
    'w256f32': dict(
        io='f32', B=1, H=16, L=2048, D=256, bias=None, mask=None, causal=False,
        bwd=True,
        workload='fp32 attention fwd+bwd, head dim 256',
    ),
    # The sibling fused kernel (selective scan), its own metric.
    'ssm': dict(
        io='f32', B=8, L=2048, Dm=1536, N=16, bwd=True,
        workload='fp32 selective scan fwd+bwd (Mamba-sized: batch 8, L 2048, '
        'd 1536, n 16, with D; delta in [0.01, 0.1], A = -(1..n))',
    ),
}

_ROUND = {'bf16': 'round_bf16', 'f16': 'round_f16'}


def _valid_lengths(B, L, round_to=0):
    """Key-padding valid lengths; `round_to` > 0 rounds each up to a
    multiple of it (a measurement line: no partial key tile at 64)."""
    rng = np.random.Generator(np.random.PCG64(SEED))
    valid = rng.integers(1024, L + 1, size=B)
    if round_to:
        valid = np.minimum(L, -(-valid // round_to) * round_to)
    return valid


def _sparse_blocks(L):
    """Keep-map of 128x128 blocks: kept with p=0.25, diagonal always kept."""
    nb = L // 128
    rng = np.random.Generator(np.random.PCG64(SEED + 7))
    blk = rng.random((nb, nb)) < 0.25
    blk[np.arange(nb), np.arange(nb)] = True
    return blk


ATTN_SOURCES = ('nxa_common.h', 'nxa_launch.h', 'nxa_fwd16.h', 'nxa_bwd16.h', 'nxa_fwd16.hip',
                'nxa_fwd16_wide.hip', 'nxa_bwd16.hip', 'nxa_bwd16_wide.hip', 'nxa_fwd.hip',
                'nxa_bwd.hip', 'nxa_attn32.hip', 'nxa_capi.hip', 'nxa_norm.hip')
SSM_SOURCES = ('nxa_common.h', 'nxa_ssm.hip')


def _src_fingerprint(names) -> str:
    """First 16 hex digits of a sha256 over the named kernel sources
    (``nitrix_amd/csrc``), names and contents in order."""
    import hashlib

    h = hashlib.sha256()
    for n in names:
        f = os.path.join(_ROOT, 'nitrix_amd', 'csrc', n)
        h.update(n.encode())
        h.update(open(f, 'rb').read() if os.path.exists(f) else b'<absent>')
    return h.hexdigest()[:16]


def _host_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        return os.cpu_count() or 1


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        return max(
            (i.get('num_threads', 1) for i in threadpool_info()
             if i.get('user_api') == 'blas'),
            default=1,
        )
    except Exception:  # pragma: no cover
        return 1


def _cpu_baseline(name, cfg, budget_s: float = 12.0):
    """Oracle fwd [+ bwd] on blocks of query rows of single (b, h) slices of
    the workload until ~budget_s of CPU time; counted FLOPs as the GPU line."""
    from oracle import attention as O

    B, H, L, D = cfg['B'], cfg['H'], cfg['L'], cfg['D']
    rnd = getattr(O, _ROUND[cfg['io']]) if cfg['io'] in _ROUND else None
    rng = np.random.Generator(np.random.PCG64(SEED + 1))
    scale = 1.0 / math.sqrt(D)
    rows = min(L, 1024)
    valid = _valid_lengths(B, L, cfg.get('round_lengths', 0)) if cfg['mask'] == 'keypad' else None
    blk = _sparse_blocks(L) if cfg['mask'] == 'blocksparse' else None
    per_pair = 14.0 * D if cfg['bwd'] else 4.0 * D

    def draw(shape):
        x = rng.standard_normal(shape, dtype=np.float32)
        return rnd(x) if rnd else x

    def sample(n):
        b = n % B
        r0 = (n * rows) % L
        q = draw((1, 1, rows, D))
        k = draw((1, 1, L, D))
        v = draw((1, 1, L, D))
        g = draw((1, 1, rows, D))
        bias = None
        mask = None
        if cfg['bias'] == 'full':
            bias = draw((1, 1, rows, L))
        elif cfg['bias'] == 'row':
            bias = draw((1, 1, 1, L))
        if cfg['mask'] == 'keypad':
            mask = (np.arange(L) < valid[b])[None, None, None, :]
        elif cfg['mask'] == 'blocksparse':
            rb = np.repeat(blk[r0 // 128:(r0 + rows) // 128], 128, axis=0)
            mask = np.repeat(rb, 128, axis=1)[None, None]
        if cfg['causal']:
            cm = (np.arange(r0, r0 + rows)[:, None] >= np.arange(L)[None, :])
            mask = cm[None, None] if mask is None else (mask & cm)
        kept = (
            float(np.broadcast_to(mask, (1, 1, rows, L)).sum())
            if mask is not None else float(rows * L)
        )
        return q, k, v, g, bias, mask, kept

    # Inputs are drawn before the clock starts; only oracle calls are timed.
    samples = [sample(i) for i in range(min(B, 4) if L > 256 else B * H)]
    flops = 0.0
    n = 0
    dt = 0.0
    while dt < budget_s:
        q, k, v, g, bias, mask, kept = samples[n % len(samples)]
        t0 = time.perf_counter()
        O.sdpa_forward(q, k, v, bias=bias, mask=mask, scale=scale)
        if cfg['bwd']:
            O.sdpa_backward(q, k, v, g, bias=bias, mask=mask, scale=scale)
        dt += time.perf_counter() - t0
        flops += per_pair * kept
        n += 1
    what = 'fwd+bwd' if cfg['bwd'] else 'fwd'
    return {
        'value': flops / dt / 1e12,
        'unit': 'TFLOP/s',
        'cores': int(_blas_threads()),
        'host_cores': _host_cores(),
        'kind': 'port',
        'sample': (
            f'{n} blocks of {rows} query rows x {L} keys of single (b,h) slices of '
            f'the {name} workload (same mask/bias/causal structure), numpy oracle '
            f'{what} in float32, {dt:.1f} s; counted FLOPs as the GPU line'
        ),
    }


class Workload:
    """Device inputs of one configuration plus its counted work."""

    def __init__(self, name, cfg, torch, dev):
        self.name, self.cfg = name, cfg
        B, H, L, D = cfg['B'], cfg['H'], cfg['L'], cfg['D']
        dtype = {'bf16': torch.bfloat16, 'f16': torch.float16}.get(cfg['io'], torch.float32)
        self.dtype = dtype
        gen = torch.Generator(device=dev)
        gen.manual_seed(SEED)

        def randn(*shape, grad=False):
            x = torch.empty(*shape, device=dev, dtype=dtype)
            flat = x.view(-1)
            step = 1 << 28
            for i in range(0, flat.numel(), step):
                n = min(step, flat.numel() - i)
                flat[i:i + n] = torch.randn(n, generator=gen, device=dev, dtype=torch.float32)
            return x.requires_grad_(grad)

        bwd = cfg['bwd']
        self.q = randn(B, H, L, D, grad=bwd)
        self.k = randn(B, H, L, D, grad=bwd)
        self.v = randn(B, H, L, D, grad=bwd)
        self.dout = randn(B, H, L, D) if bwd else None
        self.bias = None
        self.mask = None
        desc = {}
        if cfg['bias'] == 'full':
            self.bias = randn(B, H, L, L)
            desc['bias'] = f'full [{B},{H},{L},{L}] {cfg["io"]}'
        elif cfg['bias'] == 'row':
            self.bias = randn(1, H, 1, L, grad=bwd)
            desc['bias'] = f'[1,{H},1,{L}] {cfg["io"]}' + (' (with dbias)' if bwd else '')
        if cfg['mask'] == 'keypad':
            valid = _valid_lengths(B, L, cfg.get('round_lengths', 0))
            self.mask = (
                torch.arange(L, device=dev)[None, :]
                < torch.as_tensor(valid, device=dev)[:, None]
            )[:, None, None, :]
            kept = float(H * L * int(valid.sum()))
            desc['mask'] = f'key-padding [{B},1,1,{L}], valid lengths {valid.tolist()}'
        elif cfg['mask'] == 'blocksparse':
            blk = _sparse_blocks(L)
            tb = torch.as_tensor(blk, device=dev)
            self.mask = tb.repeat_interleave(128, 0).repeat_interleave(128, 1)[None, None]
            kept = float(H * int(blk.sum()) * 128 * 128)
            desc['mask'] = (
                f'block-sparse [1,1,{L},{L}] bool, {int(blk.sum())} of {blk.size} '
                f'128x128 blocks kept'
            )
        elif cfg['causal']:
            kept = float(B * H * L * (L + 1) // 2)
        else:
            kept = float(B * H * L * L)
        self.kept = kept
        self.desc = desc
        self.fwd_flops = 4.0 * D * kept
        self.step_flops = (14.0 if bwd else 4.0) * D * kept
        el = torch.empty((), dtype=dtype).element_size()
        qkvo = 4 * B * H * L * D * el
        self.fwd_bytes = qkvo + B * H * L * 4 + (
            self.bias.numel() * self.bias.element_size() if self.bias is not None else 0
        ) + (self.mask.numel() if cfg['mask'] == 'blocksparse' else 0)

    def step(self, sdpa):
        c = self.cfg
        if c['bwd']:
            for t in (self.q, self.k, self.v, self.bias):
                if t is not None:
                    t.grad = None
            out = sdpa(self.q, self.k, self.v, bias=self.bias, mask=self.mask,
                       causal=c['causal'], qk_norm=c.get('qk_norm', False), backend='hip')
            out.backward(self.dout)
        else:
            sdpa(self.q, self.k, self.v, bias=self.bias, mask=self.mask,
                 causal=c['causal'], qk_norm=c.get('qk_norm', False), backend='hip')

    def check_finite(self, torch):
        if self.cfg['bwd']:
            for t in (self.q, self.k, self.v):
                assert torch.isfinite(t.grad.float()).all(), 'non-finite gradient'


def _ssm_bytes(B, L, Dm, N):
    """Compulsory HBM bytes of one selective-scan step (fp32): forward reads
    x, delta, B, C, A, D and writes y; backward reads x, delta, dy, B, C, A, D
    and writes dx, ddelta, dB, dC, dA, dD."""
    xd = B * L * Dm * 4
    bc = B * L * N * 4
    par = (Dm * N + Dm) * 4
    fwd = 3 * xd + 2 * bc + par
    bwd = 5 * xd + 4 * bc + 2 * par
    return fwd, bwd


def _ssm_cpu_baseline(cfg, budget_s: float = 12.0):
    """Oracle forward + VJP on (1, L, 64)-channel slices of the workload until
    ~budget_s of CPU time, in the GPU line's unit."""
    from oracle import ssm as S

    L, N = cfg['L'], cfg['N']
    rng = np.random.Generator(np.random.PCG64(SEED + 3))
    dm = 64

    def sample():
        x = rng.standard_normal((1, L, dm)).astype(np.float32)
        delta = (0.01 + 0.09 / (1 + np.exp(-rng.standard_normal((1, L, dm))))).astype(np.float32)
        A = -np.repeat((np.arange(N) + 1.0)[None, :], dm, 0).astype(np.float32)
        B = rng.standard_normal((1, L, N)).astype(np.float32)
        C = rng.standard_normal((1, L, N)).astype(np.float32)
        D = rng.standard_normal((dm,)).astype(np.float32)
        dy = rng.standard_normal((1, L, dm)).astype(np.float32)
        return x, delta, A, B, C, D, dy

    samples = [sample() for _ in range(2)]
    n = 0
    dt = 0.0
    while dt < budget_s:
        x, delta, A, B, C, D, dy = samples[n % 2]
        t0 = time.perf_counter()
        S.selective_scan(x, delta, A, B, C, D)
        S.selective_scan_vjp(x, delta, A, B, C, D, dy, acc_dtype=np.float32)
        dt += time.perf_counter() - t0
        n += 1
    return {
        'value': n * L * dm / dt / 1e9,
        'unit': 'Gelem/s',
        'cores': int(_blas_threads()),
        'host_cores': _host_cores(),
        'kind': 'port',
        'sample': (
            f'{n} slices of 1 x {L} steps x {dm} channels x {N} states of the ssm workload, '
            f'numpy oracle forward + VJP in float32, {dt:.1f} s'
        ),
    }


def _bench_ssm(args, torch) -> int:
    """Selective scan fwd+bwd through the public drop-in (autograd over the
    C ABI); value = (batch, step, channel) elements per second."""
    from nitrix_amd import _lib, selective_scan

    _lib.lib()
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    cfg = CONFIGS['ssm']
    Bn, L, Dm, N = cfg['B'], cfg['L'], cfg['Dm'], cfg['N']
    gen = torch.Generator(device=dev)
    gen.manual_seed(SEED)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device=dev, dtype=torch.float32)

    x = randn(Bn, L, Dm).requires_grad_(True)
    delta = (0.01 + 0.09 * torch.sigmoid(randn(Bn, L, Dm))).requires_grad_(True)
    A = (-(torch.arange(N, device=dev, dtype=torch.float32) + 1.0)).repeat(Dm, 1)
    A.requires_grad_(True)
    Bm = randn(Bn, L, N).requires_grad_(True)
    Cm = randn(Bn, L, N).requires_grad_(True)
    Dv = randn(Dm).requires_grad_(True)
    dy = randn(Bn, L, Dm)
    leaves = (x, delta, A, Bm, Cm, Dv)

    def step():
        for t in leaves:
            t.grad = None
        y = selective_scan(x, delta, A, Bm, Cm, Dv, backend='hip')
        y.backward(dy)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
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
    elems = Bn * L * Dm
    value = elems / (ms * 1e-3) / 1e9

    prof_steps = max(3, min(args.steps, 10))
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(prof_steps):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kernels = {}
    for kname in ('ssm_fwd', 'ssm_bwd'):
        tot, n = _lib.profile_read(kname)
        if n:
            kernels[kname] = {'avg_ms': tot / n, 'launches_per_step': n / prof_steps}
    _lib.profile_reset()
    assert all(torch.isfinite(t.grad).all() for t in leaves), 'non-finite gradient'
    fwd_b, bwd_b = _ssm_bytes(Bn, L, Dm, N)
    # The backward pass (five kernels) dominates and is bound by VALU issue
    # (one exponential and a few fp32 operations per state step; its
    # compulsory bytes move at ~10 % of HBM bandwidth).  Its VALU work per
    # step is the counted instructions of its kernels (transcendentals
    # weighted 4, quarter rate) times 64 lanes, over its measured duration,
    # against 256 CUs x 4 SIMDs x 32 lanes x 2.4 GHz (the published
    # 157.3 TFLOP/s fp32 vector rate with an FMA counted as two).
    bwd_s = kernels['ssm_bwd']['avg_ms'] * 1e-3
    lane_ops = SSM_BWD_VALU_WAVE_INSTS * 64
    achieved = lane_ops / bwd_s / 1e12
    src = _src_fingerprint(SSM_SOURCES)
    roofline = {
        'kernel': 'ssm_bwd (backward pass: local, carry, chunk, two reductions)',
        'bound': 'valu',
        'achieved': round(achieved, 3),
        'peak': PEAK_VALU_TLANEOPS,
        'unit': 'Tlane-op/s',
        'frac': round(achieved / PEAK_VALU_TLANEOPS, 4),
        'traffic': None,
        'valu_source': SSM_VALU_SOURCE,
        'valu_counts_measured_at': SSM_VALU_SRC,
        'kernel_src': src,
        'compulsory_hbm_gbs': round(bwd_b / bwd_s / 1e9, 2),
    }
    if src != SSM_VALU_SRC:
        # The instruction counts were taken on other kernel sources.
        roofline['valu_counts_stale'] = True
    cpu = None if args.no_cpu_baseline else _ssm_cpu_baseline(cfg)
    line = {
        'metric': f'selective scan fwd+bwd Gelem/s at B{Bn} L{L} D{Dm} N{N} (fp32)',
        'value': round(value, 3),
        'unit': 'Gelem/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms, 4),
        'wall_s_timed': round(wall, 4),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': 'f32',
        'data': 'synthetic',
        'config': {
            'workload': cfg['workload'],
            'config_id': 'ssm',
            'B': Bn, 'L': L, 'D': Dm, 'N': N,
            'global_batch': Bn,
            'seq_len': L,
            'parallelism': 'single GPU',
        },
        'fwd_gbs': round(fwd_b / (kernels['ssm_fwd']['avg_ms'] * 1e-3) / 1e9, 2),
        'kernels': {k_: {kk: round(vv, 5) for kk, vv in v_.items()} for k_, v_ in kernels.items()},
        'roofline': roofline,
        'cpu_baseline': cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


def _measured_traffic(name: str, kernel: str) -> dict:
    """``traffic`` (HBM bytes per launch) from the committed counter profile,
    when it covers this configuration's dominant kernel."""
    hit = MEASURED_TRAFFIC.get(name)
    if hit is None or hit[0] != kernel:
        return {}
    src = _src_fingerprint(ATTN_SOURCES)
    out = {'traffic_source': TRAFFIC_SOURCE, 'traffic_measured_at': TRAFFIC_SRC,
           'kernel_src': src}
    if src == TRAFFIC_SRC:
        out['traffic'] = hit[1]
    else:
        # Measured on other kernel sources: kept beside, not reported as traffic.
        out['traffic_stale'] = hit[1]
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=20)
    ap.add_argument('--warmup', type=int, default=10)
    ap.add_argument('--config', choices=sorted(CONFIGS), default='c2')
    ap.add_argument('--no-cpu-baseline', action='store_true')
    ap.add_argument(
        '--copy-calibration',
        type=int,
        default=0,
        metavar='MIB',
        help='only run 5 device-to-device copies of MIB MiB (reference '
        'kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)',
    )
    ap.add_argument(
        '--round-lengths',
        type=int,
        default=0,
        metavar='N',
        help='key-padding configurations only: round every valid length up to '
        'a multiple of N (64: no partial key tile), a measurement line for the '
        'cost of partial tiles, not a BASELINE configuration',
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

    if args.config == 'ssm':
        return _bench_ssm(args, torch)

    from nitrix_amd import _lib, scaled_dot_product_attention

    _lib.lib()
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    name = args.config
    cfg = CONFIGS[name]
    if args.round_lengths:
        if cfg['mask'] != 'keypad' or args.round_lengths < 1:
            print('--round-lengths needs a key-padding configuration and N >= 1',
                  file=sys.stderr)
            return 2
        cfg = dict(cfg, round_lengths=args.round_lengths,
                   workload=cfg['workload'] +
                   f', valid lengths rounded up to multiples of {args.round_lengths}')
    wl = Workload(name, cfg, torch, dev)
    B, H, L, D = cfg['B'], cfg['H'], cfg['L'], cfg['D']

    def step():
        wl.step(scaled_dot_product_attention)

    # The timed steps follow the warm-up, and the per-kernel pass the timed
    # steps, directly: a pause between them (the finiteness check at the end
    # loads torch kernels on first use, ~0.2 s) lets the clocks drop, and the
    # next steps then run up to 10 % slower.
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

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
    value = wl.step_flops / (ms * 1e-3) / 1e12

    # Per-kernel durations (HIP events around each launch, same stream).
    prof_steps = max(3, min(args.steps, 10))
    _lib.profile_reset()
    _lib.profile_enable(True)
    for _ in range(prof_steps):
        step()
    torch.cuda.synchronize()
    _lib.profile_enable(False)
    kernels = {}
    for kname in ('tilemap', 'tile_order', 'fwd', 'delta', 'dkdv', 'dq', 'dbias_reduce',
                  'rms_norm_fwd', 'rms_norm_bwd'):
        tot, n = _lib.profile_read(kname)
        if n:
            kernels[kname] = {'avg_ms': tot / n, 'launches_per_step': n / prof_steps}
    _lib.profile_reset()
    wl.check_finite(torch)

    peak = PEAK_BF16_TFLOPS if cfg['io'] in ('bf16', 'f16') else PEAK_F32_TFLOPS
    per_pair = {'fwd': 4.0 * D, 'dkdv': 8.0 * D, 'dq': 6.0 * D}
    dom = max(
        (k_ for k_ in kernels if k_ in per_pair),
        key=lambda k_: kernels[k_]['avg_ms'] * kernels[k_]['launches_per_step'],
    )
    fwd_s = kernels['fwd']['avg_ms'] * 1e-3
    fwd_tflops = wl.fwd_flops / fwd_s / 1e12
    if name == 'c4':
        achieved = wl.fwd_bytes / fwd_s / 1e9
        roofline = {
            'kernel': 'fwd',
            'bound': 'hbm',
            'achieved': round(achieved, 2),
            'peak': PEAK_HBM_GBS,
            'unit': 'GB/s',
            'frac': round(achieved / PEAK_HBM_GBS, 4),
            'traffic': None,
            'algorithmic_bytes': int(wl.fwd_bytes),
        }
        roofline.update(_measured_traffic(name, 'fwd'))
    else:
        # FLOPs of one step's launches of the kernel over their summed time
        # (one launch per step except for chunked shared-bias gradients).
        dom_flops = per_pair[dom] * wl.kept
        dom_s = kernels[dom]['avg_ms'] * kernels[dom]['launches_per_step'] * 1e-3
        achieved = dom_flops / dom_s / 1e12
        roofline = {
            'kernel': dom,
            'bound': 'mfma',
            'achieved': round(achieved, 3),
            'peak': peak,
            'unit': 'TFLOP/s',
            'frac': round(achieved / peak, 4),
            'traffic': None,
        }
        roofline.update(_measured_traffic(name, dom))

    cpu = None if args.no_cpu_baseline else _cpu_baseline(name, cfg)

    what = 'fwd+bwd' if cfg['bwd'] else 'fwd'
    metric = METRIC if name == 'c2' else (
        f'attention {what} TFLOP/s and % of {cfg["io"]} MFMA peak at '
        f'B{B} H{H} L{L} D{D}' + (' (and % of HBM bandwidth)' if name == 'c4' else '')
    )
    config = {
        'workload': cfg['workload'],
        'config_id': name,
        'B': B,
        'H': H,
        'L': L,
        'D': D,
        'global_batch': B,
        'seq_len': L,
        'mask': wl.desc.get('mask'),
        'bias': wl.desc.get('bias'),
        'causal': cfg['causal'],
        'counted_tflop_per_step': round(wl.step_flops / 1e12, 4),
        'dense_equiv_tflop_per_step': round(
            (14.0 if cfg['bwd'] else 4.0) * D * B * H * L * L / 1e12, 4
        ),
        'parallelism': 'single GPU',
    }
    line = {
        'metric': metric,
        'value': round(value, 3),
        'unit': 'TFLOP/s',
        'n_gpus': 1,
        'steps': args.steps,
        'warmup': args.warmup,
        'ms_per_step': round(ms, 4),
        'wall_s_timed': round(wall, 4),
        'pct_of_peak': round(100.0 * value / peak, 3),
        'higher_is_better': True,
        'scaling': 'weak',
        'vs_baseline': None,
        'dtype': cfg['io'],
        'data': 'synthetic',
        'config': config,
        'fwd_tflops': round(fwd_tflops, 3),
        'fwd_pct_of_peak': round(100.0 * fwd_tflops / peak, 3),
        'kernels': {k_: {kk: round(vv, 5) for kk, vv in v_.items()} for k_, v_ in kernels.items()},
        'roofline': roofline,
        'cpu_baseline': cpu,
    }
    if name == 'c4':
        line['fwd_hbm_gbs'] = roofline['achieved']
        line['fwd_pct_of_hbm'] = round(100.0 * roofline['frac'], 3)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == '__main__':
    sys.exit(main())
