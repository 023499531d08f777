"""CPU tests of the factor helpers' host logic (no GPU): what feedback_factors_of_grams refuses."""

import pytest
import torch

import gptq_2d_ldl as LDL


def test_factor_pair_refuses_stream_capture(monkeypatch):
    """Under stream capture the three-stream pair raises before it touches a stream or the library (the single
    ldl_of_inverse calls are the capturable form)."""
    monkeypatch.setattr(torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: True)
    with pytest.raises(RuntimeError, match="cannot be captured"):
        LDL.feedback_factors_of_grams(torch.eye(4), torch.eye(4))
