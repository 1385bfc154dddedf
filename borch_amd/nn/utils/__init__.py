"""``borch_amd.nn.utils`` — ``fusion`` (the BN fold of the prepare step); the rest is torch's."""
import torch.nn.utils as _tu

from . import fusion  # noqa: F401


def __getattr__(name):
    return getattr(_tu, name)
