"""A whole prefill (swiftltx_amd.prefill.PrefillStep) on the small MLX-4bit
Llama of test_gpu_decode (two layers, two safetensors shards, tied lm_head),
against the same pipeline run in numpy from the oracle's functions
(LlamaModel.swift:168-203, 230-282; attention replaced on both sides by the q
rows, so every row depends on its own token only):

* the last token's logits within the parity gate (max|d|/max|ref| <= 1e-2)
  of the numpy pipeline, at prompt lengths that take the MFMA GEMM (M > 1,
  split-K included) and the GEMV (M = 1, for q|k|v and gate/up; the fused o
  and down calls run the GEMM at every M);
* row independence: the last row's logits do not depend on the other tokens;
* a captured prefill replays with new token ids exactly as an eager run.
"""
import numpy as np
import pytest

from oracle import q4_oracle as o
from test_gpu_decode import _ref_logits
from test_gpu_loader import _write_model

pytestmark = pytest.mark.gpu


def _prefill(pkg, dev, tmp_path, S, stream=None):
    from swiftltx_amd.prefill import PrefillStep
    from swiftltx_amd.weights import ModelWeights
    src = _write_model(tmp_path)
    mw = ModelWeights.from_directory(str(tmp_path), device=dev)
    return src, mw, PrefillStep(mw, S, stream=stream)


def _run(ps, ids):
    import torch
    ps.tokens.copy_(torch.tensor(ids, dtype=torch.int32))
    torch.cuda.synchronize()
    ps.forward()
    torch.cuda.synchronize()
    return ps.logits[0].float().cpu().numpy()


@pytest.mark.parametrize("S", [1, 7, 96])
def test_prefill_last_logits_match_numpy(pkg, dev, tmp_path, S):
    src, mw, ps = _prefill(pkg, dev, tmp_path, S)
    rng = np.random.default_rng(S)
    ids = rng.integers(0, mw.config.vocab_size, S).tolist()
    got = _run(ps, ids)
    ref = _ref_logits(src, ids[-1])
    err = np.max(np.abs(got - ref)) / np.max(np.abs(ref))
    assert err <= 1e-2, (S, err)
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 2e-2 * np.max(np.abs(ref)):
        assert int(np.argmax(got)) == int(np.argmax(ref)), S


def test_prefill_rows_are_independent(pkg, dev, tmp_path):
    """With the attention stand-in, row S-1 sees only its own token: the
    last logits of [a, b, ..., t] and of [t] agree (one path runs the GEMM
    throughout, the other the GEMV for q|k|v and gate/up)."""
    src, mw, ps = _prefill(pkg, dev, tmp_path, 40)
    from swiftltx_amd.prefill import PrefillStep
    one = PrefillStep(mw, 1)
    rng = np.random.default_rng(5)
    ids = rng.integers(0, mw.config.vocab_size, 40).tolist()
    a = _run(ps, ids)
    b = _run(one, ids[-1:])
    assert np.max(np.abs(a - b)) <= 1e-2 * np.max(np.abs(b)), np.max(np.abs(a - b))


def test_prefill_graph_replay(pkg, dev, tmp_path):
    """Captured once (after an eager run on the same stream), the prefill
    replays with new ids copied into its token buffer, bit-identical to an
    eager forward of those ids."""
    import torch
    s = torch.cuda.Stream()
    src, mw, ps = _prefill(pkg, dev, tmp_path, 64, stream=s)
    rng = np.random.default_rng(6)
    ps.tokens.copy_(torch.tensor(rng.integers(0, mw.config.vocab_size, 64), dtype=torch.int32))
    torch.cuda.synchronize()
    ps.capture()
    for rep in range(3):
        ids = rng.integers(0, mw.config.vocab_size, 64).tolist()
        ps.tokens.copy_(torch.tensor(ids, dtype=torch.int32))
        torch.cuda.synchronize()
        ps.replay()
        torch.cuda.synchronize()
        replayed = ps.logits[0].float().cpu().numpy().copy()
        with torch.cuda.stream(s):
            ps.forward()
        s.synchronize()
        eager = ps.logits[0].float().cpu().numpy()
        assert np.array_equal(replayed, eager), rep
        ref = _ref_logits(src, ids[-1])
        assert np.max(np.abs(eager - ref)) <= 1e-2 * np.max(np.abs(ref)), rep
