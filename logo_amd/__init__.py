"""LoGo's attention hot path on MI355X (gfx950): HIP kernels behind a C ABI
(``liblogo_hip.so``), ``torch.ops.logo_hip`` operators, and Python mirrors of
the reference's ``logo.ops`` interface and attention layer.

With the environment variable ``LOGO_OPS_ALIAS=1``, importing this package
installs the ``logo.ops`` import alias (``logo_amd.logo_ops_alias``), so the
reference's ``from logo.ops import sq_full_attn`` resolves to this build.
"""

import os as _os

if _os.environ.get("LOGO_OPS_ALIAS") == "1":
    from . import logo_ops_alias as _alias

    _alias.install()
