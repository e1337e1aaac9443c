"""Loader policy of ltc_cuda (no GPU needed): first-use build, the mtime freshness
check the reference's JIT cache performs (ltc_cuda.py:138-234), and the gfx
target check."""

from __future__ import annotations

import os
import time
import types

import ltc_cuda


def test_device_arch_strips_feature_flags():
    props = types.SimpleNamespace(gcnArchName="gfx950:sramecc+:xnack-")
    assert ltc_cuda.device_arch(props) == "gfx950"
    assert ltc_cuda.device_arch(types.SimpleNamespace(gcnArchName="gfx942")) == "gfx942"
    assert ltc_cuda.device_arch(types.SimpleNamespace()) == ""
    assert ltc_cuda.TARGET_ARCH == "gfx950"


def test_load_action_policy():
    act = ltc_cuda.load_action
    # nothing built: build on first use unless LTC_JIT=0
    assert act(False, False, "") == "build"
    assert act(False, False, "1") == "build"
    assert act(False, False, "0") == "missing"
    # built and fresh: load
    assert act(True, False, "") == "load"
    assert act(True, False, "0") == "load"
    # built but older than a source: warn by default, rebuild only when asked
    assert act(True, True, "") == "warn"
    assert act(True, True, "0") == "warn"
    assert act(True, True, "1") == "rebuild"


def test_stale_sources_compares_mtimes(tmp_path):
    lib = tmp_path / "libx.so"
    old_src, new_src = tmp_path / "a.hip", tmp_path / "b.hip"
    for f in (old_src, lib, new_src):
        f.write_text("x")
    now = time.time()
    os.utime(old_src, (now - 20, now - 20))
    os.utime(lib, (now - 10, now - 10))
    os.utime(new_src, (now, now))
    got = ltc_cuda.stale_sources(str(lib), [str(old_src), str(new_src), str(tmp_path / "gone")])
    assert got == [str(new_src)]


def test_build_script_lists_existing_sources():
    bs = ltc_cuda._build_script()
    srcs = bs.source_files()
    assert len(srcs) >= 5 and all(os.path.isfile(s) for s in srcs)
    assert any(s.endswith("ltc_capi.h") for s in srcs)
    assert "--offload-arch=gfx950" in bs.command("/tmp/x.so")
    assert "--offload-arch=gfx942" in bs.command("/tmp/x.so", "gfx942")
