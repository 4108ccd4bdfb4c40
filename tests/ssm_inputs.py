"""Test helpers: the seeded workloads of ssm_scan.synthetic plus float64 conversion."""

import torch

from ssm_scan.synthetic import baseline_inputs, triton_test_inputs  # noqa: F401


def np64(t):
    return None if t is None else t.detach().to("cpu", torch.float64).numpy()
