"""ThreadedDatasetLoader contract (models/modules/_loader.py:8-43) and the decode-only
dataset of the GPU data path; CPU only."""
import threading

import numpy as np
import pytest
import torch

from musc_hip import _loader


class Recording(torch.utils.data.Dataset):
    def __init__(self, n, fail_at=None):
        self.n, self.fail_at = n, fail_at
        self.lock = threading.Lock()
        self.max_requested = -1

    def __len__(self):
        return self.n

    def __getitem__(self, i):
        with self.lock:
            self.max_requested = max(self.max_requested, i)
        if i == self.fail_at:
            raise KeyError(f'item {i}')
        return {'x': torch.tensor([i, 2 * i]), 'i': i}


def test_order_collation_and_length():
    ds = Recording(11)
    loader = _loader.ThreadedDatasetLoader(ds, batch_size=4, workers=3, prefetch_batches=2, pin_memory=False)
    assert len(loader) == 3
    batches = list(loader)
    assert [b['i'].tolist() for b in batches] == [[0, 1, 2, 3], [4, 5, 6, 7], [8, 9, 10]]
    assert torch.equal(batches[1]['x'], torch.tensor([[4, 8], [5, 10], [6, 12], [7, 14]]))
    assert list(_loader.ThreadedDatasetLoader(Recording(0), pin_memory=False)) == []


def test_prefetch_is_bounded():
    ds = Recording(40)
    loader = _loader.ThreadedDatasetLoader(ds, batch_size=4, workers=4, prefetch_batches=2, pin_memory=False)
    for k, _ in enumerate(loader):
        # after batch k is taken, at most batch_size * prefetch_batches further items are in flight
        assert ds.max_requested < 4 * (k + 1) + 8


def test_worker_exception_reaches_the_consumer_at_its_batch():
    loader = _loader.ThreadedDatasetLoader(Recording(12, fail_at=5), batch_size=4, pin_memory=False)
    it = iter(loader)
    assert next(it)['i'].tolist() == [0, 1, 2, 3]
    with pytest.raises(KeyError, match='item 5'):
        next(it)


def test_sizes_must_be_positive():
    for kw in (dict(batch_size=0), dict(workers=0), dict(prefetch_batches=0)):
        with pytest.raises(ValueError, match='Loader sizes must be positive'):
            _loader.ThreadedDatasetLoader(Recording(3), **kw)


def test_decoded_images_and_collation(tmp_path):
    from PIL import Image
    rng = np.random.default_rng(0)
    rgb = rng.integers(0, 256, (20, 30, 3), dtype=np.uint8)
    gray = rng.integers(0, 256, (20, 30), dtype=np.uint8)
    small = rng.integers(0, 256, (8, 9, 3), dtype=np.uint8)
    paths = [str(tmp_path / n) for n in ('a.png', 'b.png', 'c.png')]
    Image.fromarray(rgb, 'RGB').save(paths[0])
    Image.fromarray(gray, 'L').save(paths[1])
    Image.fromarray(small, 'RGB').save(paths[2])
    ds = _loader.DecodedImages(paths)
    assert np.array_equal(ds[0]['image'].numpy(), rgb)
    assert np.array_equal(ds[1]['image'].numpy(), np.repeat(gray[:, :, None], 3, axis=2))   # convert('RGB')
    same = _loader.collate_images([ds[0], ds[1]])
    assert same['image'].shape == (2, 20, 30, 3) and same['image_path'] == paths[:2]
    mixed = _loader.collate_images([ds[0], ds[2]])
    assert isinstance(mixed['image'], list) and mixed['image'][1].shape == (8, 9, 3)
    loader = _loader.ThreadedDatasetLoader(ds, batch_size=2, pin_memory=False, collate_fn=_loader.collate_images)
    out = list(loader)
    assert [b['image_path'] for b in out] == [paths[:2], paths[2:]]


def test_leaving_early_cancels_queued_items():
    import time

    class Slow(Recording):
        def __getitem__(self, i):
            time.sleep(0.05)
            return super().__getitem__(i)

    ds = Slow(200)
    loader = _loader.ThreadedDatasetLoader(ds, batch_size=4, workers=2, prefetch_batches=4, pin_memory=False)
    it = iter(loader)
    assert next(it)['i'].tolist() == [0, 1, 2, 3]
    it.close()            # leaving the loop: the pool shuts down here
    # 20 items were queued (16 in flight + 4 refilled); without cancelling, every one of them
    # would be produced before the shutdown returns; with it, only the few already running
    assert ds.max_requested < 10
