"""Zero-centred RMSNorm (reference modeling/zRMSNorm.py:4-20) on MI355X.

Same module name, parameter (``weight``, zeros: the gain is ``1 + weight``), ``eps``
default and arithmetic (fp32, result in the input dtype) as the reference. The
forward and backward are one HIP row pass each (``zmoe_rmsnorm_rows``). The
transformer block normalises right before the MoE layer
(modeling/transformer_block.py:41-42); passing this module to
``MoELayer.forward(..., norm=...)`` folds that normalisation and the layer's unpad
gather into the same pass.
"""

import torch
import torch.nn as nn

from zmoe import functional as _zf


class ZeroCenteredRMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.zeros(dim))

    def forward(self, x):
        return _zf.rmsnorm_rows(x, self.weight, self.eps)

    def extra_repr(self):
        return f"{tuple(self.weight.shape)}, eps={self.eps}"
