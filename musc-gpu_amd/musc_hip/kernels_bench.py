"""Per-kernel micro-benchmarks of libmusc_hip on one GPU (used for rocprofv3 runs).

    python musc-gpu_amd/musc_hip/kernels_bench.py msm [--n 83 --p 1369 --c 1024 --iters 3 --engine fp32|split16]
                                                       [--normalize]
    python musc-gpu_amd/musc_hip/kernels_bench.py lnamd [--n 83 --layers 4 --iters 3]
    python musc-gpu_amd/musc_hip/kernels_bench.py attention [--dtype fp32|fp16 --blocks 24]
    python musc-gpu_amd/musc_hip/kernels_bench.py copy [--mib 1024 --iters 3]
    python musc-gpu_amd/musc_hip/kernels_bench.py super_fast [--n 83 --iters 3] (config 3 from tokens)
    python musc-gpu_amd/musc_hip/kernels_bench.py e2e --n 160 --iters 1       (config 5; --from-files: from PNGs)
    (msm, super_fast and e2e take --engine fp32|split16 for the MSM dot products)
    python musc-gpu_amd/musc_hip/kernels_bench.py mfma_peak                   (device calibration)
    python musc-gpu_amd/musc_hip/kernels_bench.py hbm                         (HBM calibration)
    python musc-gpu_amd/musc_hip/kernels_bench.py preprocess --n 160 [--src 1024 --files 64]  (data path)
    python musc-gpu_amd/musc_hip/kernels_bench.py msm lnamd copy --iters 1   (several in one process)

Each prints one JSON line with the average duration of the kernel(s) from HIP
events and the derived rate against the MI355X peak.  `copy` is a plain
device-to-device copy of known size, the calibration point for rocprofv3
FETCH_SIZE / WRITE_SIZE counters.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
if os.path.dirname(HERE) not in sys.path:
    sys.path.insert(0, os.path.dirname(HERE))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from musc_hip import _MSM_hip, _attention_hip, _lnamd_hip, synthetic  # noqa: E402
from musc_hip import _runtime as rt  # noqa: E402

FP32_MFMA_TFLOPS = 157.3
FP16_MFMA_TFLOPS = 2500.0
HBM_GBPS = 8000.0


def _events():
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def bench_msm(args):
    dev = torch.device('cuda:0')
    n, p, c = args.n, args.p, args.c
    engine = args.engine
    z = synthetic.msm_features(n, p, c, seed=42).to(dev)
    a, b = _MSM_hip.rank_window(n)
    _MSM_hip.check_engine(engine, p)
    ws = rt.workspace(_MSM_hip.workspace_bytes(n, p, c, engine), dev)
    scores = torch.empty((n, p), dtype=torch.float64, device=dev)
    lib, s = rt.library(), rt.stream(dev)
    t = {'prepare': [], 'pairs': [], 'refine': [], 'rank': []}
    # --normalize: rows scored as Z[i, q] / ||Z[i, q]|| inside the kernels, as the pipeline
    # scores every LNAMD pool (models/musc.py:238)
    flags = rt.MSM_NORMALIZE_ROWS if args.normalize else 0
    for it in range(args.iters + 1):
        evs = [_events() for _ in range(4)]
        evs[0][0].record()
        if engine == 'split16':
            rt.check(lib.musc_msm_split_prepare_f32(z.data_ptr(), n, p, c, flags, ws.data_ptr(), ws.numel(), s),
                     'prepare')
        else:
            rt.check(lib.musc_msm_prepare_f32(z.data_ptr(), n, p, c, flags, ws.data_ptr(), ws.numel(), s),
                     'prepare')
        evs[0][1].record()
        evs[1][0].record()
        if engine == 'split16':
            rt.check(lib.musc_msm_split_pair_minima(n, p, c, ws.data_ptr(), ws.numel(), s), 'pairs')
        else:
            rt.check(lib.musc_msm_pair_minima_f32(z.data_ptr(), n, p, c, ws.data_ptr(), ws.numel(), s), 'pairs')
        evs[1][1].record()
        evs[2][0].record()
        rt.check(lib.musc_msm_refine_f32(z.data_ptr(), n, p, c, ws.data_ptr(), ws.numel(), s), 'refine')
        evs[2][1].record()
        evs[3][0].record()
        rt.check(lib.musc_msm_rank_f32(n, p, a, b, scores.data_ptr(), ws.data_ptr(), ws.numel(), s), 'rank')
        evs[3][1].record()
        torch.cuda.synchronize()
        if it > 0:
            for k, (e0, e1) in zip(t, evs):
                t[k].append(e0.elapsed_time(e1))
        print(f'[msm] iteration {it} done', file=sys.stderr, flush=True)
    avg = {k: sum(v) / len(v) for k, v in t.items()}
    flop = float(c) * p * p * n * (n - 1)
    tf = flop / (avg['pairs'] / 1e3) / 1e12
    res = {'kernel': 'msm', 'engine': engine, 'n': n, 'p': p, 'c': c, 'normalize_rows': bool(args.normalize),
           'avg_ms': avg, 'pair_flop': flop, 'pair_tflops': tf}
    if engine == 'split16':
        # three fp16 MFMA products per fp32 dot product: the fp16 matrix-core work is 3x the
        # algorithmic FLOP; tf is the fp32-equivalent rate
        res['pair_fp16_mfma_tflops'] = 3 * tf
        res['pair_frac_fp16_mfma_peak'] = 3 * tf / FP16_MFMA_TFLOPS
    else:
        res['pair_frac_fp32_mfma_peak'] = tf / FP32_MFMA_TFLOPS
    return res


def bench_lnamd(args):
    """All layers x radii 1/3/5 in one launch: the pipeline's variant (raw window sums,
    normalised inside MSM) and the fused-L2 variant."""
    dev = torch.device('cuda:0')
    toks = [t.to(dev) for t in synthetic.pool_tokens(args.n, args.layers, seed=42)]
    radii = [1, 3, 5]
    n, L, T, C = args.n, args.layers, 1370, 1024
    nbytes = 4.0 * n * L * (T * C + len(radii) * (T - 1) * C)
    res = {'kernel': 'lnamd', 'n': n, 'layers': L, 'radii': radii, 'algorithmic_bytes': nbytes}
    for name, kw in (('raw_sums', dict(raw_sums=True)), ('fused_l2', dict(l2norm=True))):
        ts = []
        for it in range(args.iters + 1):
            e0, e1 = _events()
            e0.record()
            out = _lnamd_hip.lnamd(toks, radii, layout='rlbpc', **kw)
            e1.record()
            torch.cuda.synchronize()
            if it > 0:
                ts.append(e0.elapsed_time(e1))
            del out
            print(f'[lnamd {name}] iteration {it} done', file=sys.stderr, flush=True)
        ms = sum(ts) / len(ts)
        gbps = nbytes / (ms / 1e3) / 1e9
        res[name] = {'avg_ms': ms, 'gbps': gbps, 'frac_hbm_peak': gbps / HBM_GBPS}
    return res


def bench_super_fast(args):
    """Config 3 from layer tokens: LNAMD r=3 with the 37 -> 28 adaptive pooling in the same
    pass, MSM on the 784-patch pool (normalised rows), epilogue to 518 x 518."""
    from musc_hip import pipeline
    dev = torch.device('cuda:0')
    n = args.n
    toks = [synthetic.plumbing_tokens(n, 1370, 1024, seed=42).to(dev)]
    ts, lnamd_ms, pair_ms = [], [], []
    for it in range(args.iters + 1):
        timing = {}
        e0, e1 = _events()
        e0.record()
        pipeline.score_pool(toks, r_list=[3], image_size=518, pool_grid=28, timing=timing, msm_engine=args.engine)
        e1.record()
        torch.cuda.synchronize()
        if it > 0:
            ts.append(e0.elapsed_time(e1))
            lnamd_ms += [a.elapsed_time(b) for a, b in timing['lnamd']]
            pair_ms += [a.elapsed_time(b) for a, b in timing['pairs']]
        print(f'[super_fast] iteration {it} done', file=sys.stderr, flush=True)
    total = sum(ts) / len(ts)
    pair = sum(pair_ms) / len(pair_ms)
    lnamd = sum(lnamd_ms) / len(lnamd_ms)
    p = 784
    flop = 1024.0 * p * p * n * (n - 1)
    nbytes = 4.0 * n * (1370 * 1024 + p * 1024)     # tokens read once, pooled pool written once
    return {'kernel': 'super_fast', 'engine': args.engine, 'n': n, 'total_ms': total, 'images_per_s': n / (total / 1e3),
            'lnamd_pooled_ms': lnamd, 'lnamd_pooled_gbps': nbytes / (lnamd / 1e3) / 1e9, 'pair_ms': pair,
            'pair_tflops': flop / (pair / 1e3) / 1e12}


def _measure_library():
    """The HBM measurement probes (musc-gpu_amd/measure/libmusc_measure.so, musc_measure.h),
    built beside the product library but not part of it."""
    import ctypes
    from musc_hip import build
    lib = ctypes.CDLL(build.MEASURE_LIB)
    vp, i, ll = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong
    lib.musc_measure_hbm_stream.argtypes = [i, vp, vp, ll, vp]
    lib.musc_measure_lnamd_pattern.argtypes = [vp, vp, i, i, i, i, i, i, vp]
    lib.musc_measure_hbm_stream.restype = lib.musc_measure_lnamd_pattern.restype = i
    return lib


def bench_hbm(args):
    """Achievable HBM rates (one-shot read / write / copy of 2 GiB) and the rate of the LNAMD
    stream kernel's access pattern replayed without arithmetic at config 2's shape."""
    dev = torch.device('cuda:0')
    lib, s = _measure_library(), rt.stream(dev)
    res = {'kernel': 'hbm'}
    nbytes = 2 << 30
    src = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for mode, name, moved in ((0, 'read', nbytes), (1, 'write', nbytes), (2, 'copy', 2 * nbytes)):
        ts = []
        for it in range(args.iters + 1):
            e0, e1 = _events()
            e0.record()
            rt.check(lib.musc_measure_hbm_stream(mode, src.data_ptr(), dst.data_ptr(), nbytes, s),
                     'musc_measure_hbm_stream')
            e1.record()
            torch.cuda.synchronize()
            if it > 0:
                ts.append(e0.elapsed_time(e1))
        ms = sum(ts) / len(ts)
        res[name] = {'bytes': moved, 'avg_ms': ms, 'gbps': moved / (ms / 1e3) / 1e9,
                     'frac_hbm_peak': moved / (ms / 1e3) / 1e9 / HBM_GBPS}
        print(f'[hbm] {name} done', file=sys.stderr, flush=True)
    del src, dst
    n, L, T, C, R = 83, 4, 1370, 1024, 3
    toks = torch.zeros((L, n, T, C), dtype=torch.float32, device=dev)
    out = torch.empty((R, L, n, T - 1, C), dtype=torch.float32, device=dev)
    read_b, write_b = 4.0 * n * L * (T - 1) * C, 4.0 * n * L * R * (T - 1) * C
    # mode 0: reads and writes interleaved as in the kernel; 1: writes only; 2: reads only
    for mode, name, moved in ((0, 'lnamd_pattern', read_b + write_b), (1, 'lnamd_pattern_writes_only', write_b),
                              (2, 'lnamd_pattern_reads_only', read_b)):
        ts = []
        for it in range(args.iters + 1):
            e0, e1 = _events()
            e0.record()
            rt.check(lib.musc_measure_lnamd_pattern(toks.data_ptr(), out.data_ptr(), n, L, T, C, R, mode, s),
                     'musc_measure_lnamd_pattern')
            e1.record()
            torch.cuda.synchronize()
            if it > 0:
                ts.append(e0.elapsed_time(e1))
        ms = sum(ts) / len(ts)
        res[name] = {'bytes': moved, 'avg_ms': ms, 'gbps': moved / (ms / 1e3) / 1e9,
                     'frac_hbm_peak': moved / (ms / 1e3) / 1e9 / HBM_GBPS}
        print(f'[hbm] {name} done', file=sys.stderr, flush=True)
    return res


def bench_attention(args):
    dev = torch.device('cuda:0')
    dtype = torch.float32 if args.dtype == 'fp32' else torch.float16
    B, H, T, D = 4, 16, 1370, 64
    blocks = [tuple(x.to(dtype) for x in qkv)
              for qkv in synthetic.attention_blocks(args.blocks, B, H, T, D, device=dev)]
    # Two timings of the same back-to-back launches: GPU-paced (a spin kernel of about
    # 5 ms runs first, so that every launch is queued before the first attention kernel
    # starts and the events measure the kernels alone) and host-paced (the Python
    # wrapper's per-call overhead shows as gaps when it exceeds a kernel's duration).
    ts, ts_host = [], []
    for it in range(args.iters + 1):
        for paced in ('gpu', 'host'):
            e0, e1 = _events()
            if paced == 'gpu':
                torch.cuda._sleep(10_000_000)
            e0.record()
            for q, k, v in blocks:
                _attention_hip.attention(q, k, v, D ** -0.5)
            e1.record()
            torch.cuda.synchronize()
            if it > 0:
                (ts if paced == 'gpu' else ts_host).append(e0.elapsed_time(e1) / len(blocks))
        print(f'[attention] iteration {it} done', file=sys.stderr, flush=True)
    ms = sum(ts) / len(ts)
    ms_host = sum(ts_host) / len(ts_host)
    flop = 4.0 * B * H * T * T * D
    tf = flop / (ms / 1e3) / 1e12
    peak = FP32_MFMA_TFLOPS if dtype == torch.float32 else FP16_MFMA_TFLOPS
    return {'kernel': 'attention', 'dtype': args.dtype, 'B': B, 'H': H, 'T': T, 'D': D, 'blocks': args.blocks,
            'avg_ms_per_block': ms, 'flop_per_block': flop, 'tflops': tf, 'frac_mfma_peak': tf / peak,
            'peak_tflops': peak, 'host_paced_ms_per_block': ms_host,
            'timing': 'avg_ms_per_block: launches queued behind a spin kernel (GPU-paced); '
                      'host_paced_ms_per_block: launches issued as the Python wrapper returns'}


def bench_e2e(args):
    """Config 5: random-init ViT-L/14 at 518 px over N seeded images (5 % with an anomalous
    rectangle), tokens after blocks 6/12/18/24, LNAMD r 1/3/5, MSM, epilogue, RsCIN."""
    from musc_hip import pipeline, vit
    dev = torch.device('cuda:0')
    torch.manual_seed(0)
    model = vit.vit_l14(518).to(dev).eval()
    imgs, anomalous = synthetic.images(n=args.n, size=518, seed=42)
    imgs = imgs.to(dev)
    ts = []
    for it in range(args.iters + 1):
        timing = {}
        out = pipeline.run_category(model, imgs, timing=timing, msm_engine=args.engine)
        torch.cuda.synchronize()
        e0, e1, e2, e3 = timing['events'][0]
        if it > 0:
            ts.append((e0.elapsed_time(e1), e1.elapsed_time(e2), e2.elapsed_time(e3), e0.elapsed_time(e3)))
        print(f'[e2e] iteration {it} done', file=sys.stderr, flush=True)
        del out
    enc, score, rsc, total = (sum(t[i] for t in ts) / len(ts) for i in range(4))
    res = {'kernel': 'e2e', 'engine': args.engine, 'n': args.n, 'encoder_ms': enc, 'lnamd_msm_epilogue_ms': score,
           'rscin_ms': rsc, 'total_ms': total, 'images_per_s': args.n / (total / 1e3), 'anomalous_images': anomalous}
    if args.from_files:
        res['from_files'] = _e2e_from_files(args, model, imgs, dev)
    return res


def _e2e_from_files(args, model, imgs, dev):
    """The same images as 1024 x 1024 PNG files: threaded PIL decode, pinned uint8 batches,
    GPU preprocessing to 518 (the evaluation transform), then run_category; wall clock."""
    import tempfile

    from PIL import Image

    from musc_hip import _loader, pipeline
    from musc_hip.synthetic import CLIP_MEAN, CLIP_STD
    mean = torch.tensor(CLIP_MEAN, device=dev).view(1, 3, 1, 1)
    std = torch.tensor(CLIP_STD, device=dev).view(1, 3, 1, 1)
    rgb = ((imgs * std + mean).clamp(0, 1) * 255).round().to(torch.uint8)               # back to 8-bit RGB
    rgb = torch.nn.functional.interpolate(rgb.float(), size=(1024, 1024), mode='nearest').to(torch.uint8)
    rgb = rgb.permute(0, 2, 3, 1).contiguous().cpu().numpy()
    with tempfile.TemporaryDirectory(dir=os.environ.get('TMPDIR', '/tmp')) as d:
        paths = []
        for i in range(rgb.shape[0]):
            paths.append(os.path.join(d, f'{i:04d}.png'))
            Image.fromarray(rgb[i], 'RGB').save(paths[-1], compress_level=1)
        print('[e2e] PNG files written', file=sys.stderr, flush=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        batches = [b for b, _ in _loader.device_batches(paths, 518, batch_size=4, workers=args.workers, device=dev)]
        images = torch.cat(batches, 0)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        out = pipeline.run_category(model, images, msm_engine=args.engine)
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        del out
    return {'files': len(paths), 'source': '1024x1024 PNG', 'workers': args.workers,
            'load_decode_preprocess_s': t1 - t0, 'encoder_scoring_rscin_s': t2 - t1, 'total_s': t2 - t0,
            'images_per_s': len(paths) / (t2 - t0)}


def bench_mfma_peak(args):
    """Sustained fp32 and fp16 MFMA rates with no memory traffic (musc_calibrate_mfma_f32 / _f16)."""
    import ctypes
    dev = torch.device('cuda:0')
    blocks = 256 * 8
    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    res = {'kernel': 'mfma_peak'}
    for name, fn, peak in (('fp32', 'musc_calibrate_mfma_f32', FP32_MFMA_TFLOPS),
                           ('fp16', 'musc_calibrate_mfma_f16', FP16_MFMA_TFLOPS)):
        flop = ctypes.c_double()
        ts = []
        for it in range(args.iters + 1):
            e0, e1 = _events()
            e0.record()
            rt.check(getattr(rt.library(), fn)(out.data_ptr(), blocks, 2000, ctypes.byref(flop), rt.stream(dev)), fn)
            e1.record()
            torch.cuda.synchronize()
            if it > 0:
                ts.append(e0.elapsed_time(e1))
        ms = sum(ts) / len(ts)
        tf = flop.value / (ms / 1e3) / 1e12
        res[name] = {'avg_ms': ms, 'tflops': tf, 'frac_datasheet_peak': tf / peak}
    return res


def bench_copy(args):
    dev = torch.device('cuda:0')
    n = args.mib * (1 << 20) // 4
    src = torch.randn(n, device=dev)
    dst = torch.empty_like(src)
    ts = []
    for it in range(args.iters + 1):
        e0, e1 = _events()
        e0.record()
        dst.copy_(src)
        e1.record()
        torch.cuda.synchronize()
        if it > 0:
            ts.append(e0.elapsed_time(e1))
    ms = sum(ts) / len(ts)
    return {'kernel': 'copy', 'bytes_read': n * 4, 'bytes_written': n * 4, 'avg_ms': ms,
            'gbps_read_plus_write': 2 * n * 4 / (ms / 1e3) / 1e9}


def _synthetic_photos(n: int, h: int, w: int, seed: int = 42) -> torch.Tensor:
    """(n, h, w, 3) uint8: smooth gradients, a few rectangles and mild noise (compresses like a photo)."""
    g = torch.Generator().manual_seed(seed)
    yy = torch.linspace(0, 1, h)[:, None, None]
    xx = torch.linspace(0, 1, w)[None, :, None]
    out = torch.empty((n, h, w, 3), dtype=torch.uint8)
    for i in range(n):
        base = torch.rand((1, 1, 3), generator=g) * 160 + 40 * yy + 40 * xx
        y0, x0 = (int(v) for v in torch.randint(0, min(h, w) // 2, (2,), generator=g))
        base[y0:y0 + h // 4, x0:x0 + w // 4] += 50
        base += torch.randn((h, w, 3), generator=g) * 4
        out[i] = base.clamp(0, 255).round().to(torch.uint8)
    return out


def bench_preprocess(args):
    """Data path: decoded uint8 RGB images resident in HBM -> the encoder's normalised
    float32 batch (Pillow-exact bicubic resize + ToTensor + Normalize), against the reference's
    per-item CPU transform (PIL resize + torch ToTensor / Normalize) on host threads; with
    --files, also the whole loader (PNG decode in threads) in both forms."""
    import concurrent.futures as cf
    import os
    import tempfile

    from PIL import Image

    from musc_hip import _loader, _preprocess
    dev = torch.device('cuda:0')
    n, h, w, size = args.n, args.src, args.src, 518
    imgs = _synthetic_photos(n, h, w)
    x = imgs.to(dev)
    out = torch.empty((n, 3, size, size), dtype=torch.float32, device=dev)
    ts = []
    for it in range(args.iters + 1):
        e0, e1 = _events()
        e0.record()
        _preprocess.preprocess_u8(x, size, out=out)
        e1.record()
        torch.cuda.synchronize()
        if it > 0:
            ts.append(e0.elapsed_time(e1))
    ms = sum(ts) / len(ts)
    algo = float(n) * (h * w * 3 + 3 * size * size * 4)
    res = {'kernel': 'preprocess', 'images': n, 'src': [h, w], 'size': size, 'avg_ms': ms,
           'images_per_s': n / (ms / 1e3), 'algorithmic_bytes': algo, 'gbps': algo / (ms / 1e3) / 1e9,
           'frac_hbm_peak': algo / (ms / 1e3) / 1e9 / HBM_GBPS}
    print('[preprocess] gpu timed', file=sys.stderr, flush=True)

    mean = torch.tensor(_preprocess.OPENAI_DATASET_MEAN, dtype=torch.float32).view(-1, 1, 1)
    std = torch.tensor(_preprocess.OPENAI_DATASET_STD, dtype=torch.float32).view(-1, 1, 1)

    def cpu_transform(img: Image.Image) -> torch.Tensor:
        # the reference's per-item transform: PIL bicubic resize, ToTensor, Normalize
        r = img.resize((size, size), Image.BICUBIC)
        t = torch.from_numpy(np.array(r)).permute(2, 0, 1).contiguous().to(torch.float32).div(255)
        return t.sub(mean).div(std)

    threads = args.workers
    torch.set_num_threads(1)
    sample = min(n, 32)
    pil = [Image.fromarray(imgs[i].numpy(), 'RGB') for i in range(sample)]
    with cf.ThreadPoolExecutor(threads) as pool:
        list(pool.map(cpu_transform, pil[:threads]))
        t0 = time.perf_counter()
        cpu_out = list(pool.map(cpu_transform, pil))
        dt = time.perf_counter() - t0
    res['cpu_baseline'] = {'images_per_s': sample / dt, 'threads': threads, 'sample_images': sample,
                           'kind': 'reference transform (Pillow resize + torch ToTensor/Normalize)'}
    res['cpu_vs_gpu_max_abs_diff'] = max((cpu_out[i] - out[i].cpu()).abs().max().item() for i in range(sample))
    print('[preprocess] cpu baseline timed', file=sys.stderr, flush=True)

    if args.files:
        with tempfile.TemporaryDirectory(dir=os.environ.get('TMPDIR', '/tmp')) as d:
            paths = []
            for i in range(args.files):
                p = os.path.join(d, f'{i:04d}.png')
                Image.fromarray(imgs[i % n].numpy(), 'RGB').save(p, compress_level=1)
                paths.append(p)
            print('[preprocess] files written', file=sys.stderr, flush=True)

            class CpuItems(torch.utils.data.Dataset):
                def __len__(self):
                    return len(paths)

                def __getitem__(self, i):
                    with Image.open(paths[i]) as im:
                        return {'image': cpu_transform(im.convert('RGB')), 'image_path': paths[i]}

            t0 = time.perf_counter()
            for b in _loader.ThreadedDatasetLoader(CpuItems(), 4, threads, pin_memory=True):
                b['image'].to(dev, non_blocking=True)
            torch.cuda.synchronize()
            t_cpu = time.perf_counter() - t0
            t0 = time.perf_counter()
            for batch, _ in _loader.device_batches(paths, size, batch_size=4, workers=threads, device=dev):
                pass
            torch.cuda.synchronize()
            t_gpu = time.perf_counter() - t0
            res['loader'] = {'files': len(paths), 'format': 'PNG', 'workers': threads,
                             'cpu_transform_images_per_s': len(paths) / t_cpu,
                             'gpu_transform_images_per_s': len(paths) / t_gpu}
            print('[preprocess] loaders timed', file=sys.stderr, flush=True)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('kernels', nargs='+', choices=['msm', 'lnamd', 'super_fast', 'attention', 'copy', 'e2e',
                                                     'mfma_peak', 'hbm', 'preprocess'])
    ap.add_argument('--n', type=int, default=83)
    ap.add_argument('--p', type=int, default=1369)
    ap.add_argument('--c', type=int, default=1024)
    ap.add_argument('--layers', type=int, default=4)
    ap.add_argument('--dtype', choices=['fp32', 'fp16'], default='fp32')
    ap.add_argument('--blocks', type=int, default=24)
    ap.add_argument('--mib', type=int, default=1024)
    ap.add_argument('--iters', type=int, default=3)
    ap.add_argument('--engine', choices=['fp32', 'split16'], default='fp32', help='MSM dot-product engine')
    ap.add_argument('--normalize', action='store_true', help='msm: normalise rows in the kernels (the pipeline\'s use)')
    ap.add_argument('--src', type=int, default=1024, help='preprocess: source image side')
    ap.add_argument('--workers', type=int, default=4, help='preprocess: host threads (the reference loader uses 4)')
    ap.add_argument('--files', type=int, default=0, help='preprocess: also time the loaders over this many PNG files')
    ap.add_argument('--from-files', action='store_true',
                    help='e2e: also run the pipeline from 1024x1024 PNG files (decode, GPU preprocessing, scoring)')
    args = ap.parse_args()
    table = {'msm': bench_msm, 'lnamd': bench_lnamd, 'super_fast': bench_super_fast, 'attention': bench_attention,
             'copy': bench_copy, 'e2e': bench_e2e, 'mfma_peak': bench_mfma_peak, 'hbm': bench_hbm,
             'preprocess': bench_preprocess}
    for name in args.kernels:
        print(json.dumps(table[name](args)), flush=True)


if __name__ == '__main__':
    main()
