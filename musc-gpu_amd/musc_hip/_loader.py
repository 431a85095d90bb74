"""Bounded, ordered image loading for the GPU data path.

`ThreadedDatasetLoader` keeps the contract of the reference's loader
(models/modules/_loader.py:8-43, used for the GPU backends at models/musc.py:171-175):
dataset items are produced by a thread pool, at most batch_size * prefetch_batches
items are in flight, batches come out in dataset order, are collated like
torch's DataLoader and pinned when pin_memory is set; a worker's exception surfaces
in the consumer at its item, and leaving the iteration shuts the pool down (items
still queued are cancelled; the reference waits for them).

The GPU variant of the data path moves the per-pixel work off the host:
`DecodedImages` items are the decoded uint8 RGB arrays only (PIL decode and
`.convert("RGB")`, as datasets/mvtec.py:101, in the worker threads), and
`device_batches` copies each pinned uint8 batch to the GPU and runs the evaluation
transform there (`_preprocess.preprocess_u8`: bicubic resize, ToTensor, Normalize,
bit-identical to the CPU transform), so the host decodes and the bytes that cross
PCIe are a quarter of the float32 batch.
"""
from __future__ import annotations

import collections
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

from . import _preprocess


def _pin(obj):
    if isinstance(obj, torch.Tensor):
        return obj.pin_memory()
    if isinstance(obj, dict):
        return {k: _pin(v) for k, v in obj.items()}
    if isinstance(obj, (list, tuple)):
        return type(obj)(_pin(v) for v in obj)
    return obj


class ThreadedDatasetLoader:
    def __init__(self, dataset, batch_size: int = 4, workers: int = 4, prefetch_batches: int = 2,
                 pin_memory: bool = True, collate_fn=None):
        if batch_size < 1 or workers < 1 or prefetch_batches < 1:
            raise ValueError('Loader sizes must be positive')
        self.dataset = dataset
        self.batch_size = batch_size
        self.workers = workers
        self.prefetch_batches = prefetch_batches
        self.pin_memory = pin_memory
        self.collate_fn = collate_fn or torch.utils.data.default_collate

    def __len__(self) -> int:
        return -(-len(self.dataset) // self.batch_size)

    def __iter__(self):
        total = len(self.dataset)
        depth = self.batch_size * self.prefetch_batches
        with ThreadPoolExecutor(max_workers=self.workers) as pool:
            window: collections.deque = collections.deque()
            issued = 0

            def top_up():
                nonlocal issued
                while issued < total and len(window) < depth:
                    window.append(pool.submit(self.dataset.__getitem__, issued))
                    issued += 1

            try:
                top_up()
                while window:
                    take = min(self.batch_size, len(window))
                    samples = [window.popleft().result() for _ in range(take)]
                    top_up()
                    batch = self.collate_fn(samples)
                    yield _pin(batch) if self.pin_memory else batch
            finally:
                # leaving early (break, exception): queued items are dropped, running ones finish
                for future in window:
                    future.cancel()


class DecodedImages(torch.utils.data.Dataset):
    """Items {'image': (H, W, 3) uint8 RGB tensor, 'image_path': path} decoded with PIL."""

    def __init__(self, paths):
        self.paths = list(paths)

    def __len__(self) -> int:
        return len(self.paths)

    def __getitem__(self, idx):
        from PIL import Image
        path = self.paths[idx]
        with Image.open(path) as im:
            arr = np.array(im.convert('RGB'))            # writable copy, (H, W, 3) uint8
        return {'image': torch.from_numpy(arr), 'image_path': path}


def collate_images(samples):
    """Stack same-sized images into (B, H, W, 3); keep a list when the sizes differ."""
    imgs = [s['image'] for s in samples]
    same = all(t.shape == imgs[0].shape for t in imgs)
    return {'image': torch.stack(imgs, 0) if same else imgs, 'image_path': [s['image_path'] for s in samples]}


def device_batches(paths, size=518, batch_size: int = 4, workers: int = 4, prefetch_batches: int = 2,
                   device=None, mean=_preprocess.OPENAI_DATASET_MEAN, std=_preprocess.OPENAI_DATASET_STD):
    """Yield (images (B, 3, S, S) float32 on `device`, paths) for image files, in order."""
    device = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
    loader = ThreadedDatasetLoader(DecodedImages(paths), batch_size, workers, prefetch_batches, pin_memory=True,
                                   collate_fn=collate_images)
    for batch in loader:
        img = batch['image']
        if isinstance(img, torch.Tensor):
            out = _preprocess.preprocess_u8(img.to(device, non_blocking=True), size, mean, std)
        else:
            out = torch.stack([_preprocess.preprocess_u8(t.to(device, non_blocking=True), size, mean, std)
                               for t in img], 0)
        yield out, batch['image_path']
