"""Dtype table and the API-compatible runtime tuner.

Reference: flashdp/core/utils.py:5-47, flashdp/layers/utils.py:14-17.
"""
from __future__ import annotations

import torch

# input dtype -> (accumulation dtype, output dtype...) as in the reference table.
# int8 is listed by the reference but unreachable (its forward is a float GEMM);
# the HIP kernels take fp32, fp16 and bf16.
supported_acc_dtypes = {
    torch.float16: (torch.float32, torch.float16),
    torch.bfloat16: (torch.float32, torch.bfloat16),
    torch.float32: (torch.float32,),
}


class RuntimeAutoTuner:
    """Keeps the reference's interface (flashdp/core/utils.py:15-47).

    The reference times a Triton path against a TorchScript path with
    ``time.time()`` and keeps the faster one, so its choice (and result) varies
    from run to run.  Here there is exactly one implementation per operator --
    the HIP kernel -- so ``choose_function`` always returns the first candidate
    and no calls are spent on timing.  Arguments are accepted and recorded.
    """

    def __init__(self, enable=True, warmup_iterations=10, measure_iterations=100, log=False) -> None:
        self.enable = enable
        self.if_final_tune = False
        self.chosen_func = None
        self.warmup_iterations = warmup_iterations
        self.measure_iterations = measure_iterations
        self.log = log

    def choose_function(self, funcs_list, *args, **kwargs):
        self.chosen_func = funcs_list[0]
        if self.log:
            print(f"Chosen function: {self.chosen_func}")
        return self.chosen_func

    def final_tune(self):
        self.if_final_tune = True
