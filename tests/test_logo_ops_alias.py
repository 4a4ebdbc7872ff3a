"""The ``logo.ops`` import alias (logo_amd/logo_ops_alias.py) on the CPU.

A stand-in parent package named ``logo`` (written to a temporary directory by
this test; it holds only a module that imports the way the reference's
attention layer does, ``from logo.ops import sq_full_attn``,
logo/layers/logo.py:29) shows that, with the alias installed, the reference's
import lines resolve to this build's objects without editing them.
"""

import os
import subprocess
import sys
import textwrap

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CALLER = textwrap.dedent("""
    from logo.ops import (SelInfo, assert_close, build_selection, get_abs_err, get_err_ratio, sdpa_causal_ref,
                          sq_full_attn, sq_full_attn_dense_ref)
    from logo.ops.common import SelInfo as SelInfo2
    from logo.ops.selected_full_attn import sq_full_attn as sq2
    from logo.ops.dense_full_attn import sq_full_attn_dense_ref as dref2
    import logo.ops
    """)

CHECK = textwrap.dedent("""
    import sys
    {setup}
    import logo.layers_standin as L
    import logo_amd.ops as ops
    import logo_amd.ops.common as common
    assert L.sq_full_attn is ops.sq_full_attn and L.sq2 is ops.sq_full_attn
    assert L.SelInfo is common.SelInfo and L.SelInfo2 is common.SelInfo
    assert L.dref2 is ops.sq_full_attn_dense_ref and L.build_selection is ops.build_selection
    assert L.logo.ops.sq_full_attn is ops.sq_full_attn
    assert sys.modules["logo.ops"].__logo_amd_target__ == "logo_amd.ops"
    try:
        import logo.ops.triton_utils
    except ImportError as e:
        assert "not served" in str(e)
    else:
        raise AssertionError("logo.ops.triton_utils should not import")
    print("alias ok")
    """)


def _standin(tmp_path):
    pkg = tmp_path / "logo"
    pkg.mkdir()
    (pkg / "__init__.py").write_text('"""stand-in parent package for the alias test"""\n')
    (pkg / "layers_standin.py").write_text(CALLER)
    return str(tmp_path)


def _run(tmp_path, setup, env_extra=None):
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([_standin(tmp_path), ROOT])
    env.update(env_extra or {})
    return subprocess.run([sys.executable, "-c", CHECK.format(setup=setup)], env=env, capture_output=True,
                          text=True, timeout=300)


def test_alias_by_install_call(tmp_path):
    r = _run(tmp_path, "import logo_amd.logo_ops_alias as a; a.install()")
    assert r.returncode == 0 and "alias ok" in r.stdout, r.stderr


def test_alias_by_environment(tmp_path):
    r = _run(tmp_path, "import logo_amd", {"LOGO_OPS_ALIAS": "1"})
    assert r.returncode == 0 and "alias ok" in r.stdout, r.stderr


def test_install_refuses_after_the_real_module(tmp_path):
    """A logo.ops that was imported before the hook (here a stand-in's own)
    makes install() raise instead of leaving two operator sets in use."""
    root = _standin(tmp_path)
    (tmp_path / "logo" / "ops").mkdir()
    (tmp_path / "logo" / "ops" / "__init__.py").write_text("sq_full_attn = None\n")
    code = ("import logo.ops\nimport logo_amd.logo_ops_alias as a\ntry:\n    a.install()\nexcept RuntimeError as e:\n"
            "    print('refused', e)\n")
    env = dict(os.environ, PYTHONPATH=os.pathsep.join([root, ROOT]))
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "refused" in r.stdout, r.stderr
