"""GEMM kernel choices for the LM step on MI355X.

The LM's GEMMs (in_proj, the fused f/i/x projection, out_proj and the tied
head, forward and backward) go through torch's hipBLASLt / rocBLAS calls.
PyTorch's TunableOp can time every library solution for each GEMM shape and
keep the fastest; ``tunableop_mi355x_lm.csv`` holds that choice for the C5
shapes (batch 8 x 2048 tokens, d_model 768, d_inner 1536, N 64, vocab 50257),
made on this image's ROCm / hipBLASLt versions (the file's validator lines;
TunableOp ignores a file whose validators do not match the running stack).

``load()`` turns TunableOp on with tuning off and reads the file: listed
shapes use the recorded solution, every other shape the library's default.
``tune(path)`` turns tuning on, so the next calls time the solutions of
shapes not yet listed and record them in ``path``.
"""
import os

import torch

DEFAULT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tunableop_mi355x_lm.csv")


def load(path=DEFAULT):
    """Use the recorded GEMM choices; returns whether the file was read."""
    import torch.cuda.tunable as tun
    if not torch.cuda.is_available() or not os.path.exists(path):
        return False
    tun.enable(True)
    tun.tuning_enable(False)
    return bool(tun.read_file(path))


def tune(path, max_iterations=30):
    """Time and record the solutions of GEMM shapes met from now on."""
    import torch.cuda.tunable as tun
    tun.enable(True)
    tun.tuning_enable(True)
    tun.set_max_tuning_iterations(max_iterations)
    tun.set_filename(path)
