"""Serve ``logo.ops`` from this build, so the reference's callers need no edit.

The reference's attention layer imports its operator with
``from logo.ops import sq_full_attn`` (logo/layers/logo.py:29), and its
package ``logo/ops/__init__.py:4-23`` exports ``sq_full_attn``,
``sq_full_attn_dense_ref``, ``sdpa_causal_ref``, ``build_selection``,
``SelInfo``, ``get_abs_err``, ``get_err_ratio`` and ``assert_close`` from the
submodules ``selected_full_attn``, ``dense_full_attn`` and ``common``.

``install()`` puts an import hook at the front of ``sys.meta_path`` that
answers those module names with this build's modules:

====================================  =====================================
name the reference imports            served by
====================================  =====================================
``logo.ops``                          ``logo_amd.ops``
``logo.ops.selected_full_attn``       ``logo_amd.ops.sq_attn``
``logo.ops.dense_full_attn``          ``logo_amd.ops.dense``
``logo.ops.common``                   ``logo_amd.ops.common``
====================================  =====================================

Each alias is a module object of its own name whose attributes are the
served module's (the same function and class objects), so ``logo.ops`` is a
package, its submodules import normally and the rest of the ``logo`` package
(the model, the cache, the layers) stays the reference's.  Call it once,
before anything imports ``logo``::

    import logo_amd.logo_ops_alias
    logo_amd.logo_ops_alias.install()
    from logo import LoGoForCausalLM   # its layers now call logo_amd's kernels

or set ``LOGO_OPS_ALIAS=1`` and ``import logo_amd`` first.  Names that the
hook does not serve (``logo.ops.triton_utils``, the reference's Triton
helpers) raise ``ImportError`` once it is installed: nothing in this build
runs Triton.  ``uninstall()`` removes the hook and the alias modules.
"""

import importlib
import importlib.abc
import importlib.machinery
import sys

__all__ = ["ALIASES", "install", "uninstall", "installed"]

ALIASES = {
    "logo.ops": "logo_amd.ops",
    "logo.ops.selected_full_attn": "logo_amd.ops.sq_attn",
    "logo.ops.dense_full_attn": "logo_amd.ops.dense",
    "logo.ops.common": "logo_amd.ops.common",
}


class _AliasLoader(importlib.abc.Loader):
    def __init__(self, target):
        self.target = target

    def create_module(self, spec):
        return None  # a fresh module object named after the alias

    def exec_module(self, module):
        src = importlib.import_module(self.target)
        for key, val in vars(src).items():
            if not (key.startswith("__") and key.endswith("__")):
                setattr(module, key, val)
        module.__doc__ = src.__doc__
        if hasattr(src, "__all__"):
            module.__all__ = list(src.__all__)
        module.__logo_amd_target__ = self.target


class _AliasFinder(importlib.abc.MetaPathFinder):
    def find_spec(self, fullname, path=None, target=None):
        if fullname in ALIASES:
            is_pkg = fullname == "logo.ops"
            return importlib.machinery.ModuleSpec(fullname, _AliasLoader(ALIASES[fullname]), is_package=is_pkg)
        if fullname.startswith("logo.ops."):
            raise ImportError(f"{fullname} is not served by logo_amd (its logo.ops alias covers "
                              f"{', '.join(sorted(ALIASES))})")
        return None


_FINDER = _AliasFinder()


def installed():
    return _FINDER in sys.meta_path


def install():
    """Answer imports of ``logo.ops`` and its submodules with this build's
    modules.  Raises if the reference's own ``logo.ops`` was already imported
    (its Triton kernels would stay bound in the modules that imported it)."""
    for name in ALIASES:
        mod = sys.modules.get(name)
        if mod is not None and getattr(mod, "__logo_amd_target__", None) is None:
            raise RuntimeError(f"{name} is already imported from {getattr(mod, '__file__', '?')}: "
                               "install the logo_amd alias before importing logo")
    if not installed():
        sys.meta_path.insert(0, _FINDER)


def uninstall():
    if installed():
        sys.meta_path.remove(_FINDER)
    for name in ALIASES:
        mod = sys.modules.get(name)
        if mod is not None and getattr(mod, "__logo_amd_target__", None) is not None:
            del sys.modules[name]
