"""Sampler.scores (engine/sampler.py:30-52, qvex_sampler_scores on the device)
against the float64 restatement used to pin the fused kernel's oracle: same
kept set, same log-probs to fp32 accuracy (GPU); the filter settings follow the
reference's rules (CPU)."""

import numpy as np
import pytest
import torch

from qvex.sampler import Sampler, SamplingParams
from test_oracle_spec_filter import ref_scores


@pytest.mark.gpu
@pytest.mark.parametrize("T,top_k,top_p,pen", [(0.7, 20, 0.95, 0.0), (0.6, 10, 0.8, 1.5), (1.0, 5, 1.0, 0.0),
                                               (0.0, 20, 0.95, 2.0), (0.7, 100, 0.9, 0.0), (0.8, 0, 0.7, 0.5)])
def test_scores_mirror_reference(T, top_k, top_p, pen):
    g = np.random.default_rng(int(T * 10) + top_k)
    V = 512
    logits = (g.standard_normal(V) * 2.0).astype(np.float32)
    seen = (g.random(V) < 0.2).astype(np.float32)
    s = Sampler(SamplingParams(temperature=T, top_k=top_k, top_p=top_p, presence_penalty=pen), V)
    if pen:
        s.seen = torch.from_numpy(seen).to("cuda:0")
    got = s.scores(torch.from_numpy(logits).to("cuda:0"),
                   extra_seen=[3] if pen else None).cpu().numpy().astype(np.float64)
    ref = ref_scores(logits, T, seen if pen else None, pen, top_k if T > 0 else 0, top_p, extra=(3,) if pen else ())
    assert np.array_equal(np.isfinite(got), np.isfinite(ref))
    fin = np.isfinite(ref)
    np.testing.assert_allclose(got[fin], ref[fin], rtol=1e-5, atol=1e-5)


def test_filter_settings_follow_the_reference():
    """engine/sampler.py:44-50: top-k when 0 < top_k < V (top_k >= V or 0 means the
    whole vocabulary is the candidate set), top-p when 0 < top_p < 1; greedy
    sampling ignores both."""
    s = Sampler(SamplingParams(temperature=0.7, top_k=0, top_p=0.9), 1000)
    assert (s.top_k, s.top_p) == (0, 0.9)
    s = Sampler(SamplingParams(temperature=0.7, top_k=100, top_p=0.9), 1000)
    assert (s.top_k, s.top_p) == (100, 0.9)
    s = Sampler(SamplingParams(temperature=0.7, top_k=1000, top_p=1.0), 1000)
    assert (s.top_k, s.top_p) == (0, 1.0)
    assert Sampler(SamplingParams(temperature=0.0, top_k=20, top_p=0.9), 1000).top_k == 0
    s = Sampler(SamplingParams(), 248320)                                     # the reference's defaults
    assert (s.top_k, s.top_p) == (20, 0.95)
