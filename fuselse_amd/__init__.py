"""fuselse_amd: row-wise log-sum-exp kernels for AMD Instinct MI355X (gfx950).

``fuselse_amd.ext`` is the extension object carrying the reference's function
names; ``make_fuselse_logsumexp(fuselse_amd.ext, robust=True)`` builds the
torch.logsumexp drop-in.  The kernels live in ``libfuselse_amd.so`` behind the
C ABI declared in ``include/fuselse_amd.h``.
"""

from . import ext
from .autograd import make_fuselse_logsumexp
from .selective import make_selective_log_softmax

__all__ = ["ext", "make_fuselse_logsumexp", "make_selective_log_softmax", "logsumexp", "selective_log_softmax"]


_default = None


def logsumexp(input, dim=-1, keepdim=False):
    """torch.logsumexp drop-in with the robust forward (reference default)."""
    global _default
    if _default is None:
        _default = make_fuselse_logsumexp(ext, robust=True)
    return _default(input, dim=dim, keepdim=keepdim)


_default_sls = None


def selective_log_softmax(logits, index):
    """trl.trainer.utils.selective_log_softmax drop-in: one fused pass for CUDA
    fp32 logits, robust special values."""
    global _default_sls
    if _default_sls is None:
        _default_sls = make_selective_log_softmax(ext, robust=True)
    return _default_sls(logits, index)
