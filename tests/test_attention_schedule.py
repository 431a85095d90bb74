"""CPU model of the fp16 attention kernel's key-block schedule (csrc/attention.hip,
attn_fwd_f16_kernel).

The kernel's unrolled "whole" steps load K and V blocks through a buffer resource
with the extent of a full 32-key block and skip the ragged-key mask.  That is only
in bounds when every block such a step names is full; otherwise keys past t - 1 are
read from memory (past the end of a packed (T, B, 3E) tensor for the last heads).
The model below restates which blocks a pair of whole steps names and checks, for
every sequence length 1..2048, that all of them are full.  The loop bound it models
is read from the kernel source, so a change there that the model does not follow
fails here first.
"""
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, 'musc-gpu_amd', 'csrc', 'attention.hip')
KB = 32


def _whole_pairs(t: int, bound: str) -> list[int]:
    """kb of every pair of whole steps the kernel runs for sequence length t."""
    nkb = -(-t // KB)
    limit = {'nfull': t // KB, 'nkb': nkb}[bound]
    kbs, kb = [], 0
    while kb + 4 < limit:
        kbs.append(kb)
        kb += 2
    return kbs


def _blocks_named(kb: int) -> set[int]:
    # step kb: K load kb+3, V load kb+1, unmasked logits kb+2; step kb+1: K load kb+4,
    # V load kb+2, unmasked logits kb+3
    return {kb + 3, kb + 1, kb + 2, kb + 4}


def _violations(bound: str) -> list[tuple[int, int]]:
    bad = []
    for t in range(1, 2049):
        for kb in _whole_pairs(t, bound):
            for blk in _blocks_named(kb):
                if (blk + 1) * KB > t:
                    bad.append((t, blk))
    return bad


def test_kernel_source_matches_model():
    src = open(SRC).read()
    body = src[src.index('attn_fwd_f16_kernel('):]
    body = body[:body.index('l_run = halves_sum(l_run);')]
    assert re.search(r'const int nfull = t / KB;', body)
    assert re.search(r'for \(; kb \+ 4 < nfull; kb \+= 2\) \{\s*step\(kb, sa, base_a, sb, pfa, pfb, Whole\{\}\);'
                     r'\s*step\(kb \+ 1, sb, base_b, sa, pfb, pfa, Whole\{\}\);', body)
    # the whole step's loads and unchecked softmax block, as the model names them
    assert 'load_block(kg, kb + 3, std::integral_constant<bool, kFull>{})' in body
    assert 'load_block(vg, kb + 1, std::integral_constant<bool, kFull>{})' in body
    assert 'part_a(kb + 2, s_new, b_new, pf_make, NoCheck{})' in body


def test_whole_steps_touch_only_full_blocks():
    assert _violations('nfull') == []


def test_model_detects_the_unbounded_schedule():
    # the bound the kernel had before (kb + 4 < nkb) lets K block kb + 4 be the ragged
    # last block, e.g. at t = 150, 257 and 1370 (the ViT-L/14 sequence length)
    bad = _violations('nkb')
    ts = {t for t, _ in bad}
    assert {150, 257, 1370} <= ts
    assert all((blk + 1) * KB > t and blk == -(-t // KB) - 1 for t, blk in bad)
