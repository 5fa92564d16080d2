"""Population-forward throughput on one MI355X: member-tokens/s at 1024 members x 2048 tokens.

Workload (the reference's EGGROLL population evaluation, train/val/eggroll.py:130-146, on one GPU):
  model     the fixed 37.7M GPT (utils/model.py), make_model init seed 0 on the CPU (eggroll.py:38-53)
  tokens    one 2049-token sequence ~ Zipf(s=1.1) over [0, 4096) (torch.multinomial, CPU generator seed 0),
            shared by every member (eggroll.py:143); x = seq[:-1], y = seq[1:]
  members   512 antithetic pairs = 1024 members, sigma 0.002 (eggroll.py:31), rank-1 noise on the 48 block
            matrices, sliced from the seed-0 noise buffer at the step-0 offsets (eggroll.py:114-128)
A step = offsets draw + noise regeneration + weight prep + the fused population forward -> 1024 losses.
The CPU baseline is the fp32 oracle restatement of the same forward on a bounded member sample.

--workload orthogonal-fp32-head: the large-population variant, 2048 members = 1024 orthogonal antithetic
pairs (Hadamard draws of run.py:223-238 mapped to weight space, noise_amd.eggroll.orthogonal_directions)
with the fp32 head as split-bf16x3; a step = orthogonal draws + the forward in two 1024-member chunks.
"""
import argparse
import json
import os
import sys
import time

TOKENS = 2048
PAIRS = 512
SIGMA = 0.002
BF16_PEAK = 2.5e15           # MI355X dense bf16 MFMA, FLOP/s
HBM_PEAK = 8.0e12            # MI355X HBM3E, B/s
WINDOWS = None


def zipf_tokens(n, s=1.1, vocab=4096, seed=0):
    import torch
    p = (torch.arange(vocab, dtype=torch.float64) + 1) ** -s
    return torch.multinomial(p / p.sum(), n, replacement=True, generator=torch.Generator().manual_seed(seed))


def visible_pairs(T, window):
    """Sum over queries of keys visible under q >= k, q - k <= window."""
    return sum(min(q, window) + 1 for q in range(T))


def kernel_flops_per_launch(name, label, members, T):
    """Algorithmic FLOPs one launch performs (dense products; rank-1 terms not counted)."""
    rows = members * T
    if name == 'noise_pop_qkv':
        return 2 * 512 * 1536 * rows
    if name == 'noise_pop_fc':
        return 2 * 512 * 2048 * rows
    if name == 'noise_pop_residual':
        return 2 * (2048 if label == 'mlp.c_proj' else 512) * 512 * rows
    if name == 'noise_pop_mlp':
        return 2 * 2 * 512 * 2048 * rows
    if name in ('noise_pop_attn_mlp', 'noise_pop_block'):
        return 2 * (512 * 512 + 2 * 512 * 2048) * rows
    if name == 'noise_pop_block_qkv':
        return 2 * (512 * 512 + 2 * 512 * 2048 + 512 * 1536) * rows
    if name == 'noise_pop_head_ce':
        return 2 * 512 * 4096 * rows
    if name == 'noise_attention_fwd':
        window = int(label.split()[-1])
        return 4 * 64 * 8 * members * visible_pairs(T, window)
    return None


PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'profiles', 'population_forward_1024x2048.md')
# entry point (bench label) -> the kernel name in the committed trace of the default workload (the block
# kernels that form the next block's q/k/v: 4 of their 7 launches carry value embeddings)
ROCPROF_NAME = {'noise_pop_qkv': 'qkv16_kernel<false>', 'noise_pop_head_ce': 'head_x_kernel<false, false>',
                'noise_pop_block_qkv[block]': 'block_kernel<true, 3, false, 2, 0>',
                'noise_pop_block[block]': 'block_kernel<false, 0, false, 0, 0>'}


def profiled_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 summary (FETCH_SIZE + WRITE_SIZE, scaled
    by the 1 GiB copy calibration), or None."""
    name = ROCPROF_NAME.get(kernel) or ('attention_vt_kernel<true, false>' if kernel.startswith('noise_attention') else None)
    if not name or not os.path.exists(PROFILE):
        return None
    for line in open(PROFILE):
        cells = [c.strip() for c in line.strip().strip('|').split('|')]
        if len(cells) == 7 and cells[0] == name:
            try:
                return int((float(cells[5]) + float(cells[6])) * 1e9)
            except ValueError:
                return None
    return None


def profiled_mfma_busy(kernel):
    """The kernel's MFMA-busy fraction from the committed counter table (SQ_VALU_MFMA_BUSY_CYCLES over the
    cycles it ran, on its own clock), or None."""
    name = ROCPROF_NAME.get(kernel) or ('attention_vt_kernel<true, false>' if kernel.startswith('noise_attention') else None)
    if not name or not os.path.exists(PROFILE):
        return None
    col = None
    for line in open(PROFILE):
        cells = [c.strip() for c in line.strip().strip('|').split('|')]
        if 'MFMA busy' in cells:
            col = cells.index('MFMA busy')   # the counter table's header
        elif col is not None and len(cells) > col and cells[0] == name:
            try:
                return float(cells[col])
            except ValueError:
                return None
    return None


def block_matrix_names():
    return [f'transformer.h.{i}.{s}.weight' for i in range(8)
            for s in ('attn.c_q', 'attn.c_k', 'attn.c_v', 'attn.c_proj', 'mlp.c_fc', 'mlp.c_proj')]


def host_cpu():
    """Model name, physical cores and hardware threads of this host (lscpu), for the CPU baselines."""
    import subprocess
    info = dict(model=None, physical_cores=None, threads=os.cpu_count())
    try:
        out = subprocess.run(['lscpu'], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return info
    kv = {}
    for line in out.splitlines():
        if ':' in line:
            k, v = line.split(':', 1)
            kv[k.strip()] = v.strip()
    info['model'] = kv.get('Model name')
    try:
        info['physical_cores'] = int(kv['Core(s) per socket']) * int(kv['Socket(s)'])
    except (KeyError, ValueError):
        pass
    return info


CPU_RUNS = 5  # timed runs of each CPU baseline after one warmup run; the median is reported


def _median_time(fn, runs=CPU_RUNS):
    """One warmup call, then the median wall time of `runs` calls (and the last call's result)."""
    out = fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        out = fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], out


def cpu_forward_config1(threads=None):
    """The reference's CPU plumbing case: the fixed model's fp32 forward + mean next-token CE (the oracle's
    restatement of utils/model.py:193-209) on a batch of 4 x 2048 tokens ~ U[0, 4096) from a CPU generator
    seeded 0, shifted by one (eggroll.py:217-229). One warmup, then the median of 5 runs."""
    import torch
    from noise_amd.model import make_model
    from oracle import model as om
    if threads:
        torch.set_num_threads(threads)
    P = {k: v.float() for k, v in make_model('cpu', 0).state_dict().items()}
    batch = torch.randint(0, 4096, (4, TOKENS + 1), generator=torch.Generator().manual_seed(0))
    x, y = batch[:, :-1], batch[:, 1:]
    with torch.no_grad():
        dt, loss = _median_time(lambda: om.gpt_forward(P, x, y))
    return dict(value=round(x.numel() / dt, 1), unit='tokens/s', loss=round(float(loss), 6), seconds=round(dt, 3),
                threads=torch.get_num_threads(), runs=f'1 warmup + median of {CPU_RUNS}',
                batch='4 x 2048 tokens ~ U[0, 4096), seed 0')


def cpu_baseline(P, tables, x, y, members):
    """The oracle forward (fp32, torch CPU) on `members` members of the same workload: one warmup run, then
    the median of 5 timed runs."""
    import torch
    from oracle import model as om
    threads = torch.get_num_threads()
    noise = {}
    for n, (a, b) in tables.items():
        noise[n] = (a[:members // 2].cpu().repeat_interleave(2, 0), b[:members // 2].cpu().repeat_interleave(2, 0))
    sign = torch.tensor([SIGMA, -SIGMA]).repeat(members // 2)
    Pc = {k: v.cpu().float() for k, v in P.items()}
    with torch.no_grad():
        dt, losses = _median_time(lambda: om.population_loss(Pc, noise, sign, x.cpu(), y.cpu(), members_per_chunk=2))
    return dict(value=members * x.numel() / dt, unit='member-tokens/s', cores=threads, kind='port',
                sample=f'{members} members x {x.numel()} tokens, fp32 oracle forward (oracle/model.py), one warmup '
                       f'run then the median of {CPU_RUNS} runs ({dt:.1f} s each) on {threads} threads',
                host=host_cpu()), losses


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=5)
    ap.add_argument('--warmup', type=int, default=2)
    ap.add_argument('--workload', choices=('population', 'orthogonal-fp32-head', 'update', 'head-error', 'dust-block',
                                           'dust-rerun', 'dust-direct', 'attention', 'lowrank', 'cpu-forward'),
                    default='population')
    ap.add_argument('--pairs', type=int, default=None,
                    help='update workload: antithetic pairs (default 512; the reference trains with 131072)')
    ap.add_argument('--update-chunk', type=int, default=8192, help='update workload: directions per GEMM pass')
    ap.add_argument('--members', type=int, default=None,
                    help='population size (default 1024; 2048 for orthogonal-fp32-head)')
    ap.add_argument('--cpu-members', type=int, default=8,
                    help='members of the CPU-baseline sample, timed 6 times: about 20 s of CPU work (0: skip)')
    ap.add_argument('--profile-steps', type=int, default=1, help='extra timed steps with per-kernel events')
    ap.add_argument('--copy-calibration', action='store_true',
                    help='only copy 1 GiB device to device (scale reference for rocprofv3 FETCH_SIZE / WRITE_SIZE)')
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        src = torch.ones(2 ** 28, device='cuda')
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps(dict(copy_bytes=2 ** 30)))
        return
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures one GPU: the library has no multi-GPU path (members would shard across GPUs with '
              'one all_gather of the per-member losses). Run with --gpus 1.', file=sys.stderr)
        sys.exit(2)

    if args.workload == 'update':
        return bench_update(args)
    if args.workload == 'head-error':
        return bench_head_error(args)
    if args.workload == 'dust-block':
        return bench_dust_block(args)
    if args.workload == 'dust-rerun':
        return bench_dust_rerun(args)
    if args.workload == 'dust-direct':
        return bench_dust_direct(args)
    if args.workload == 'attention':
        return bench_attention(args)
    if args.workload == 'lowrank':
        return bench_lowrank(args)
    if args.workload == 'cpu-forward':
        return bench_cpu_forward(args)
    import torch
    from noise_amd import eggroll as eg
    from noise_amd.model import make_model, window_sizes

    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    model = make_model('cpu', 0)
    P = {k: v.to(dev) for k, v in model.state_dict().items()}
    model = model.to(dev)
    seq = zipf_tokens(TOKENS + 1)
    x, y = seq[:-1].to(dev), seq[1:].to(dev)
    names = block_matrix_names()
    orthogonal = args.workload == 'orthogonal-fp32-head'
    members = args.members or (4 * PAIRS if orthogonal else 2 * PAIRS)
    pairs = members // 2
    chunk = min(members, 2 * PAIRS)   # members per population_forward call
    es = eg.Eggroll(model, pairs)
    rope = None
    sign = torch.tensor([SIGMA, -SIGMA], device=dev).repeat(pairs)
    directions = torch.arange(0, members, 2, device=dev) % (2 * pairs) // 2
    shapes = {n: tuple(P[n].shape) for n in names}

    gather_events = None   # (start, end) events around the noise-slice regeneration, in the profiling steps

    def step():
        if orthogonal:
            tables = eg.orthogonal_directions(shapes, pairs, seed=0, device=dev)
            W = eg.Weights(P, fp32_head=True)
            return eg.orthogonal_population(W, tables, x, y, sigma=SIGMA, chunk=chunk), tables
        offsets = es.offsets(0)
        if gather_events is not None:
            # the GPU spins briefly first, so the host has queued the launch and both events before the start
            # event runs: the interval is the kernel's own time, not the host's launch latency after a sync
            if hasattr(torch.cuda, '_sleep'):
                torch.cuda._sleep(2_000_000)
            ev = (torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            ev[0].record()
        tables = es.noise_tables({n: offsets[n] for n in names}, directions)
        if gather_events is not None:
            ev[1].record()
            gather_events.append(ev)
        W = eg.Weights(P)
        return eg.population_forward(W, tables, sign, x, y, dir_div=2, rope=rope), tables

    for _ in range(args.warmup):
        losses, tables = step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        losses, tables = step()
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    value = members * TOKENS / dt

    # per-kernel HIP events (torch's current stream = the launch stream) over extra timed steps
    timer = eg.KernelTimer()
    eg.set_timer(timer)
    gather_events = []
    for _ in range(args.profile_steps):
        step()
    torch.cuda.synchronize()
    eg.set_timer(None)
    kernels = {}
    for (name, label), (n, ms) in timer.totals().items():
        key = name if label is None else f'{name}[{label}]'
        flops = kernel_flops_per_launch(name, label, chunk, TOKENS)
        entry = dict(launches=n // args.profile_steps, ms_per_step=round(ms / args.profile_steps, 4))
        if flops is not None:
            tf = flops * n / (ms * 1e-3)
            entry.update(tflops=round(tf / 1e12, 1), mfma_frac=round(tf / BF16_PEAK, 4))
        kernels[key] = entry
    if gather_events:
        # the noise regeneration replacing the reference's buffer gather (eggroll.py:114, 126-127): one
        # noise_gather_slice_groups launch for the 48 perturbed matrices, writing their directions' a and b rows
        # in fp32
        ms = sum(s_.elapsed_time(e_) for s_, e_ in gather_events) / len(gather_events)
        written = 4 * len(directions) * sum(sum(shapes[n]) for n in names)
        kernels['noise_gather_slice_groups'] = dict(launches=1, ms_per_step=round(ms, 4), bytes_written=written,
                                              gbps=round(written / ms / 1e6, 1),
                                              hbm_frac=round(written / ms / 1e6 / (HBM_PEAK / 1e9), 4))
    timed = [k for k in kernels if 'tflops' in kernels[k]]
    roofline = None
    if timed:
        dominant = max(timed, key=lambda k: kernels[k]['ms_per_step'])
        dk = kernels[dominant]
        roofline = dict(bound='mfma', kernel=dominant, achieved=round(dk['tflops'], 1), peak=BF16_PEAK / 1e12,
                        unit='TFLOP/s', frac=dk['mfma_frac'], traffic=profiled_traffic(dominant),
                        counter_mfma_busy=profiled_mfma_busy(dominant),
                        flops_per_launch=kernel_flops_per_launch(*(dominant.rstrip(']').split('[') + [None])[:2],
                                                                 chunk, TOKENS))

    algo_flops = 68_318_208 * members * TOKENS
    if orthogonal:
        metric = 'member-tokens/sec forward at 2048 members (1024 orthogonal pairs), fp32 head, T=2048 on 1 GPU'
        workload = ('large population, fp32 head: fixed 37.7M GPT (seed-0 init), 2048 members (1024 orthogonal '
                    'antithetic pairs of Hadamard draws, sigma 0.002, rank-1 on the 48 block matrices) x 2048 '
                    'Zipf(1.1) tokens, head fp32 as split-bf16x3, fused per-member CE')
    else:
        metric = 'member-tokens/sec forward at P=1024,T=2048 on 1 GPU; attn/GEMM % MFMA peak'
        workload = ('population fitness: fixed 37.7M GPT (seed-0 init), 1024 members (512 antithetic pairs, '
                    'sigma 0.002, rank-1 noise on the 48 block matrices) x 2048 Zipf(1.1) tokens, fused '
                    'per-member CE')
    line = dict(
        metric=metric,
        value=round(value, 1), unit='member-tokens/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(dt * 1e3, 3), higher_is_better=True, scaling='weak', vs_baseline=None, dtype='bf16',
        data='synthetic',
        config=dict(workload=workload, members=members, tokens=TOKENS, pairs=pairs,
                    head='fp32 (split-bf16x3)' if orthogonal else 'bf16'),
        roofline=roofline,
        whole_forward=dict(algorithmic_tflops=round(algo_flops / dt / 1e12, 1),
                           mfma_frac=round(algo_flops / dt / BF16_PEAK, 4)),
        kernels=kernels,
        losses=dict(mean=round(losses.mean().item(), 6), first=round(losses[0].item(), 6),
                    finite=bool(torch.isfinite(losses).all().item())),
    )
    if args.cpu_members:
        cb, cpu_losses = cpu_baseline(P, {n: t for n, t in tables.items()}, x, y, args.cpu_members)
        # the reference's CPU plumbing configuration (fixed model, 4 x 2048 tokens, plain forward + mean CE)
        cb['config1_forward'] = cpu_forward_config1()
        line['cpu_baseline'] = cb
        line['cpu_parity_max_abs'] = float((cpu_losses - losses[:args.cpu_members].cpu()).abs().max())
    else:
        line['cpu_baseline'] = None
    print(json.dumps(line), flush=True)


def bench_update(args):
    """EGGROLL's update reassembly (eggroll.py:151-165) for the fixed model: fitness weights, then every
    parameter's -(1/F) sum_d w_d a_d b_d^T with the noise regenerated in-kernel. A step is one update from
    losses already resident on the GPU."""
    import torch
    from noise_amd.eggroll import Eggroll
    from noise_amd.model import make_model
    dev = torch.device('cuda', 0)
    torch.cuda.set_device(dev)
    model = make_model('cpu', 0).to(dev)
    pairs = args.pairs or PAIRS
    es = Eggroll(model, pairs)
    offsets = es.offsets(0)
    g = torch.Generator().manual_seed(0)
    losses = (8.3 + 0.01 * torch.randn(2 * pairs, generator=g)).to(dev)
    for _ in range(args.warmup):
        es.update(losses, offsets, chunk=args.update_chunk)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        grads = es.update(losses, offsets, chunk=args.update_chunk)
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / args.steps
    big = sum(p.shape[0] * p.shape[1] for p in es.params.values()
              if p.dim() == 2 and p.shape[0] % 256 == 0 and p.shape[1] % 256 == 0)
    algo = 2 * pairs * sum(p.numel() for p in es.params.values())
    executed = 3 * 2 * pairs * big  # split-bf16x3 products of the GEMM path
    print(json.dumps(dict(
        metric='EGGROLL update reassembly: gradient TFLOP/s (2 x pairs x parameters) on 1 GPU',
        value=round(algo / dt / 1e12, 2), unit='TFLOP/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(dt * 1e3, 3), higher_is_better=True, scaling='weak', vs_baseline=None,
        dtype='fp32 (split-bf16x3 MFMA)', data='synthetic',
        config=dict(workload=f'update of the fixed 37.7M GPT (60 parameters) from {2 * pairs} member losses, '
                             f'{pairs} directions regenerated in-kernel, chunk {args.update_chunk}',
                    pairs=pairs, chunk=args.update_chunk),
        executed_mfma=dict(tflops=round(executed / dt / 1e12, 1), frac=round(executed / dt / BF16_PEAK, 4)),
        grad_finite=bool(all(torch.isfinite(t).all().item() for t in grads.values())),
    )), flush=True)


def bench_head_error(args):
    """DUST.head_error (run.py:380-389) on the cached logits of one DUST batch: 8 sequences x 2048 tokens x
    4096 bf16 logits -> fp32 coordinate differences. HBM-bound: 8 KiB read + 16 KiB written per token."""
    import torch
    from noise_amd.dust import head_error
    dev = torch.device('cuda', 0)
    g = torch.Generator().manual_seed(0)
    logits = (torch.randn(8, 2048, 4096, generator=g) * 5).to(torch.bfloat16).to(dev)
    y = torch.randint(0, 4096, (8, 2048), generator=g).to(dev)
    for _ in range(args.warmup):
        head_error(logits, y, 4096)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        out = head_error(logits, y, 4096)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    traffic = 8 * 2048 * 4096 * (2 + 4)
    print(json.dumps(dict(
        metric='DUST head error (coordinate differences) throughput, tokens/s on 1 GPU', value=round(8 * 2048 / ms * 1e3),
        unit='tokens/s', n_gpus=1, steps=args.steps, warmup=args.warmup, ms_per_step=round(ms, 4),
        higher_is_better=True, scaling='weak', vs_baseline=None, dtype='fp32 (bf16 logits in)', data='synthetic',
        config=dict(workload='DUST head_error over cached bf16 logits [8, 2048, 4096]'),
        roofline=dict(bound='hbm', achieved=round(traffic / ms / 1e6, 1), peak=8000.0, unit='GB/s',
                      frac=round(traffic / ms / 1e6 / 8000.0, 4), traffic=None),
        finite=bool(torch.isfinite(out).all().item()))), flush=True)


def bench_dust_block(args):
    """DUST's block_forward (run.py:102-117) as rerun calls it: block 1 (value embeddings, window 1024) of the
    fixed model over 128 sequences (16 draws x 8 sequences) x 2048 tokens with bf16 jitter at mlp.c_fc."""
    import torch
    from noise_amd.dust import block_forward
    from noise_amd.model import make_model, rotary_tables, window_sizes
    dev = torch.device('cuda', 0)
    P = {k: v.to(dev) for k, v in make_model('cpu', 0).state_dict().items()}
    pre = 'transformer.h.1.'
    w = dict(q=P[pre + 'attn.c_q.weight'], k=P[pre + 'attn.c_k.weight'], v=P[pre + 'attn.c_v.weight'],
             gate=P[pre + 'attn.ve_gate.weight'], proj=P[pre + 'attn.c_proj.weight'], fc=P[pre + 'mlp.c_fc.weight'],
             out=P[pre + 'mlp.c_proj.weight'])
    S, T = 128, 2048
    g = torch.Generator().manual_seed(0)
    x = torch.randn(S, T, 512, generator=g).to(dev)
    ve = torch.randn(S, T, 512, generator=g).bfloat16().to(dev)
    fc = (0.1 * (torch.randint(0, 2, (S, T, 2048), generator=g) * 2 - 1)).bfloat16().to(dev)
    cos, sin = (t.to(dev) for t in rotary_tables(T))
    win = window_sizes(8)[1]
    for _ in range(args.warmup):
        block_forward(x, w, ve, cos, sin, win, fc=fc)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        out = block_forward(x, w, ve, cos, sin, win, fc=fc)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    gemm = 2 * (512 * 1536 + 512 * 512 + 2 * 512 * 2048)
    attn = 4 * 64 * 8 * visible_pairs(T, win) / T
    flops = (gemm + attn) * S * T
    print(json.dumps(dict(
        metric='DUST block_forward throughput (one block, jitter at mlp.c_fc), sequence-tokens/s on 1 GPU',
        value=round(S * T / ms * 1e3), unit='tokens/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(ms, 3), higher_is_better=True, scaling='weak', vs_baseline=None, dtype='bf16',
        data='synthetic', config=dict(workload=f'block 1 of the fixed 37.7M GPT over {S} x {T} tokens, window {win}'),
        roofline=dict(bound='mfma', achieved=round(flops / ms / 1e9, 1), peak=BF16_PEAK / 1e12, unit='TFLOP/s',
                      frac=round(flops / ms / 1e9 / (BF16_PEAK / 1e12), 4), traffic=None),
        finite=bool(torch.isfinite(out).all().item()))), flush=True)


def bench_dust_rerun(args):
    """DUST.rerun (run.py:256-279) as direct_errors calls it: 16 draws x 8 sequences x 2048 tokens rerun from block
    0 with bf16 jitter (+-0.1) at its mlp.c_fc, then blocks 1-7, the final norm and the fp32 head with per-token CE.
    The capture state (block 0's input, x0, the embedding and value-embedding outputs) is formed with torch from
    the seed-0 model and uniform tokens. Timed: `rerun` (the blocks after the jittered one on the population
    kernels) and, for comparison, `rerun_tiled` (every block on noise_dust_block)."""
    import torch
    import torch.nn.functional as F
    from types import SimpleNamespace
    from noise_amd import dust as ndust
    from noise_amd.model import make_model, window_sizes
    dev = torch.device('cuda', 0)
    n, b, T = 16, 8, TOKENS
    model = make_model('cpu', 0).to(dev)
    g = torch.Generator().manual_seed(0)
    rows = torch.randint(0, 4096, (b, T + 1), generator=g).to(dev)
    x, y = rows[:, :-1].contiguous(), rows[:, 1:].contiguous()
    with torch.no_grad():
        emb = model.transformer.wte.weight[x].float()
        x0 = F.rms_norm(emb, (512,))
        block0 = model.resid_lambdas[0] * x0 + model.x0_lambdas[0] * x0
        outputs = {'transformer.wte': emb}
        for key, table in model.value_embeds.items():
            outputs[f'value_embeds.{key}'] = table.weight[x].float()
    weights = [dict(q=blk.attn.c_q.weight, k=blk.attn.c_k.weight, v=blk.attn.c_v.weight,
                    gate=blk.attn.ve_gate.weight if blk.attn.ve_gate is not None else None,
                    proj=blk.attn.c_proj.weight, fc=blk.mlp.c_fc.weight, out=blk.mlp.c_proj.weight)
               for blk in model.transformer.h]
    state = SimpleNamespace(model=model, length=T, batch=b, outputs=outputs, blocks={0: block0}, x0=x0, x=x, y=y,
                            weights=weights)
    jit = {'transformer.h.0.mlp.c_fc': (0.1 * (torch.randint(0, 2, (n * b, T, 2048), generator=g) * 2 - 1))
           .bfloat16().to(dev)}
    timings = {}
    for name in ('rerun', 'rerun_tiled'):
        fn = getattr(ndust, name)
        with torch.no_grad():
            for _ in range(args.warmup):
                loss = fn(state, n, 0, jit)
            torch.cuda.synchronize()
            s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            s.record()
            for _ in range(args.steps):
                loss = fn(state, n, 0, jit)
            e.record()
            torch.cuda.synchronize()
        timings[name] = (s.elapsed_time(e) / args.steps, loss.clone())
    ms, loss = timings['rerun']
    # per-kernel HIP events over one more call: the population kernels of the blocks after the entry (and the
    # rest of the call: the jittered entry block, the mixing and the copies)
    from noise_amd import eggroll as eg
    timer = eg.KernelTimer()
    eg.set_timer(timer)
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.no_grad():
        s.record()
        ndust.rerun(state, n, 0, jit)
        e.record()
    torch.cuda.synchronize()
    eg.set_timer(None)
    kernels = {}
    for (kname, label), (cnt, kms) in timer.totals().items():
        kernels[kname if label is None else f'{kname}[{label}]'] = dict(launches=cnt, ms=round(kms, 4))
    kernels['other (entry block, mixing, copies)'] = dict(ms=round(s.elapsed_time(e) - sum(
        v['ms'] for v in kernels.values()), 4))
    wins = window_sizes(8)
    gemm = 2 * (512 * 1536 + 512 * 512 + 2 * 512 * 2048)
    flops = sum(gemm + 4 * 64 * 8 * visible_pairs(T, w) / T for w in wins) + 2 * 512 * 4096
    flops *= n * b * T
    tiled_ms, tiled_loss = timings['rerun_tiled']
    print(json.dumps(dict(
        metric='DUST rerun throughput from block 0 (jitter at mlp.c_fc, 8 blocks + fp32 head), sequence-tokens/s',
        value=round(n * b * T / ms * 1e3), unit='tokens/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(ms, 3), higher_is_better=True, scaling='weak', vs_baseline=None, dtype='bf16',
        data='synthetic', config=dict(workload=f'{n} draws x {b} sequences x {T} tokens from block 0 of the fixed '
                                               '37.7M GPT, fp32 head'),
        ms_per_block=round(ms / 8, 3), tiled_ms_per_step=round(tiled_ms, 3), tiled_ms_per_block=round(tiled_ms / 8, 3),
        speedup_vs_tiled=round(tiled_ms / ms, 3),
        roofline=dict(bound='mfma', achieved=round(flops / ms / 1e9, 1), peak=BF16_PEAK / 1e12, unit='TFLOP/s',
                      frac=round(flops / ms / 1e9 / (BF16_PEAK / 1e12), 4), traffic=None),
        kernels=kernels,
        mean_loss=round(loss.mean().item(), 6), max_abs_vs_tiled=float((loss - tiled_loss).abs().max()),
        mean_abs_vs_tiled=float((loss.mean(-1) - tiled_loss.mean(-1)).abs().max()),
        finite=bool(torch.isfinite(loss).all().item()))), flush=True)


def bench_dust_direct(args):
    """DUST.direct_errors (run.py:332-378) as a step calls it for one block's sites: entry block 3, sites mlp.c_fc
    (live units only) and attn.c_proj, 32 orthogonal draws in 2 reruns of 16 (nrep 16), 8 sequences x 2048 tokens,
    sigma 0.1. The capture state is synthetic (normed random block input, random c_fc outputs for the live mask):
    the work per call does not depend on its values."""
    import torch
    import torch.nn.functional as F
    from types import SimpleNamespace
    from noise_amd import dust as ndust
    from noise_amd.model import make_model
    from noise_amd.noise import OrthogonalDraws
    dev = torch.device('cuda', 0)
    b, T, draws, nrep, entry = 8, TOKENS, 32, 16, 3
    model = make_model('cpu', 0).to(dev)
    g = torch.Generator(device=dev).manual_seed(0)
    x = torch.randint(0, 4096, (b, T), device=dev, generator=g)
    y = torch.randint(0, 4096, (b, T), device=dev, generator=g)
    with torch.no_grad():
        emb = model.transformer.wte.weight[x].float()
        x0 = F.rms_norm(emb, (512,))
        block = F.rms_norm(torch.randn(b, T, 512, device=dev, generator=g), (512,))
    outputs = {'transformer.wte': emb, f'transformer.h.{entry}.mlp.c_fc': torch.randn(b, T, 2048, device=dev, generator=g),
               f'transformer.h.{entry}.attn.c_proj': torch.randn(b, T, 512, device=dev, generator=g)}
    weights = [dict(q=blk.attn.c_q.weight, k=blk.attn.c_k.weight, v=blk.attn.c_v.weight,
                    gate=blk.attn.ve_gate.weight if blk.attn.ve_gate is not None else None,
                    proj=blk.attn.c_proj.weight, fc=blk.mlp.c_fc.weight, out=blk.mlp.c_proj.weight)
               for blk in model.transformer.h]
    draw = OrthogonalDraws(seed=0, device=dev)
    state = SimpleNamespace(model=model, length=T, batch=b, outputs=outputs, blocks={entry: block}, x0=x0, x=x, y=y,
                            weights=weights, clean_loss=8.3 + 0.1 * torch.randn(b, T, device=dev, generator=g),
                            dtype=torch.bfloat16, recipe=SimpleNamespace(nrep=nrep), alpha={}, estimates={}, fits={},
                            prior_sites=[],
                            orthogonal_noise=lambda *a: draw(*a, dtype=torch.bfloat16))
    sites = [f'transformer.h.{entry}.mlp.c_fc', f'transformer.h.{entry}.attn.c_proj']
    with torch.no_grad():
        for _ in range(args.warmup):
            ndust.direct_errors(state, sites, draws, 0.1, entry=entry)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(args.steps):
            out = ndust.direct_errors(state, sites, draws, 0.1, entry=entry)
        e.record()
        torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    print(json.dumps(dict(
        metric='DUST direct_errors throughput (2 sites of block 3, 32 draws in reruns of 16), sequence-token-draws/s',
        value=round(draws * b * T / ms * 1e3), unit='token-draws/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(ms, 3), higher_is_better=True, scaling='weak', vs_baseline=None, dtype='bf16',
        data='synthetic', config=dict(workload=f'{draws} draws x {b} sequences x {T} tokens from block {entry} of the '
                                               'fixed 37.7M GPT, sites mlp.c_fc (live units) and attn.c_proj'),
        ms_per_rerun=round(ms / (draws // nrep), 3),
        finite=bool(all(torch.isfinite(v).all().item() for v in out.values())))), flush=True)


def bench_attention(args):
    """Causal attention alone through the attention(q, k, v, window) drop-in (utils/model.py:24-31): bf16 q, k,
    v [B=16, H=8, T=2048, D=64] ~ N(0, 1) from one CPU generator seeded 0 (q, k, v in order), passed as the
    [B, T, H, D] views the reference's attention takes, window = T (causal), scale 1/8. Algorithmic work 4 D
    FLOPs per visible (query, key) pair: 16 x 8 x 2,098,176 x 256 = 68.75 GFLOP per call."""
    import torch
    from noise_amd.model import attention
    dev = torch.device('cuda', 0)
    g = torch.Generator().manual_seed(0)
    B, H, T, D = 16, 8, 2048, 64
    q, k, v = (torch.randn(B, H, T, D, generator=g).bfloat16().to(dev).transpose(1, 2) for _ in range(3))
    for _ in range(args.warmup):
        attention(q, k, v, T)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        out = attention(q, k, v, T)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    flops = 4 * D * B * H * visible_pairs(T, T)
    print(json.dumps(dict(
        metric='causal attention forward TFLOP/s, bf16 [16, 8, 2048, 64] on 1 GPU', value=round(flops / ms / 1e9, 1),
        unit='TFLOP/s', n_gpus=1, steps=args.steps, warmup=args.warmup, ms_per_step=round(ms, 4),
        higher_is_better=True, scaling='weak', vs_baseline=None, dtype='bf16', data='synthetic',
        config=dict(workload='causal attention, q/k/v [16, 8, 2048, 64] bf16 ~ N(0,1) seed 0, scale 1/8, through '
                             'the attention(q, k, v, window) drop-in'),
        roofline=dict(bound='mfma', achieved=round(flops / ms / 1e9, 1), peak=BF16_PEAK / 1e12, unit='TFLOP/s',
                      frac=round(flops / ms / 1e9 / (BF16_PEAK / 1e12), 4), traffic=None, flops_per_launch=flops),
        finite=bool(torch.isfinite(out.float()).all().item()))), flush=True)


def bench_lowrank(args):
    """The antithetic perturbed linear alone through the lowrank drop-in (eggroll.py:56-58): X bf16 [2048, 512]
    and W bf16 [2048 out, 512 in] ~ N(0, 0.02^2) from one CPU generator seeded 0; 256 pairs (512 members),
    sigma 1e-3; a, b per pair sliced from the seed-0 noise buffer at offsets ~ U[0, 2^28 - 2560) from a cuda
    generator seeded 0. Output [512, 2048, 2048] fp32 in autocast's form (8.6 GB): bound by its HBM writes."""
    import torch
    from noise_amd.eggroll import lowrank
    from noise_amd.noise import DeviceGenerator
    dev = torch.device('cuda', 0)
    g = torch.Generator().manual_seed(0)
    X = torch.randn(2048, 512, generator=g).bfloat16().to(dev)
    W = (torch.randn(2048, 512, generator=g) * 0.02).bfloat16().to(dev)
    pairs, sigma, NOISE = 256, 1e-3, 2 ** 28
    offs = torch.randint(0, NOISE - 2560, (pairs,), device=dev, generator=torch.Generator(dev).manual_seed(0))
    rows = DeviceGenerator(0, dev).take(NOISE).gather(offs, 2560)
    a, b = rows[:, :2048], rows[:, 2048:]
    sign = torch.tensor([sigma, -sigma], device=dev).repeat(pairs)
    xm = X[None].expand(2 * pairs, 2048, 512)
    for _ in range(args.warmup):
        y = lowrank(xm, W, a, b, sign, dir_div=2)
        del y
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        y = lowrank(xm, W, a, b, sign, dir_div=2)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    written = y.numel() * 4
    print(json.dumps(dict(
        metric='antithetic perturbed linear output GB/s, 512 members x [2048, 2048] on 1 GPU',
        value=round(written / ms / 1e6, 1), unit='GB/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
        ms_per_step=round(ms, 4), higher_is_better=True, scaling='weak', vs_baseline=None,
        dtype='bf16 product, fp32 rank-1 and output', data='synthetic',
        config=dict(workload='lowrank drop-in: X [2048, 512] shared, W [2048, 512], 256 antithetic pairs, '
                             'sigma 1e-3, output [512, 2048, 2048] fp32'),
        roofline=dict(bound='hbm', achieved=round(written / ms / 1e6, 1), peak=HBM_PEAK / 1e9, unit='GB/s',
                      frac=round(written / ms / 1e6 / (HBM_PEAK / 1e9), 4), traffic=None),
        finite=bool(torch.isfinite(y[::97]).all().item()))), flush=True)


def bench_cpu_forward(args):
    """The reference's CPU plumbing configuration alone (no GPU): fixed model, seed-0 init, forward + mean
    next-token CE on 4 x 2048 uniform tokens, fp32 torch CPU ops (the oracle's restatement of utils/model.py)."""
    r = cpu_forward_config1()
    print(json.dumps(dict(metric='reference CPU forward tokens/s (fixed 37.7M model, batch 4 x 2048)',
                          value=r['value'], unit='tokens/s', n_gpus=0, steps=3, warmup=1, higher_is_better=True,
                          vs_baseline=None, dtype='fp32', data='synthetic', config=dict(workload=r['batch']),
                          loss=r['loss'], host=host_cpu(), threads=r['threads'])), flush=True)


if __name__ == '__main__':
    main()
