"""Op registrations of the LTV path (reference: ``nanochat/ops/__init__.py``).

Importing this package defines the ``nanochat_cuda`` ops of the reference path
and the ``nanochat_amd`` fast-path ops.  The native library is loaded lazily on
the first call, so importing works on a machine without a GPU.
"""

from nanochat_amd.ops import ltv_cuda_ops  # noqa: F401
from nanochat_amd.ops import ltv_hm_fast  # noqa: F401
