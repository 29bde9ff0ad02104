"""The backend raises the host's own exception classes.

light-vllm's step handler catches *its* ``KVCacheError`` around compact and
re-raises ``ExecutionError`` (src/light_vllm/runtime/execution/worker.py:
316-323), and its engine maps ``ExecutionNotReadyError`` / ``ExecutionError``
(src/light_vllm/runtime/engine/core.py:89-94).  These tests bind stand-in
host classes and check that every kind of raise site in the package raises
them, that no module bypasses the binding, and that light-vllm's classes are
bound on import when its modules are importable.
"""

from __future__ import annotations

import re
import subprocess
import sys
import textwrap
from pathlib import Path
from types import SimpleNamespace

import pytest
import torch

import light_vllm_amd as lv
from light_vllm_amd import errors, native
from light_vllm_amd.backend import HipPagedAttention
from light_vllm_amd.facts import facts_of
from light_vllm_amd.paged_cache import PagedKVCache, _compact_plan, dtype_code, hip_block_copy, hip_compact
from light_vllm_amd.plan import StepPlan

PACKAGE = Path(lv.__file__).resolve().parent
CPU = torch.device("cpu")


class HostKVCacheError(RuntimeError):
    pass


class HostCapacityError(HostKVCacheError):
    pass


class HostExecutionError(RuntimeError):
    pass


class HostNotReadyError(HostExecutionError):
    pass


@pytest.fixture
def host_classes():
    errors.bind(kv_cache_error=HostKVCacheError, kv_cache_capacity_error=HostCapacityError,
                execution_error=HostExecutionError, not_ready_error=HostNotReadyError)
    try:
        yield
    finally:
        errors.bind()


def _metadata(tables=((0, 1),), computed=(3,)):
    return lv.PagedAttentionMetadata(block_tables=tables, num_computed_tokens=computed,
                                     query_layouts=tuple(lv.linear_query_layout(1) for _ in tables))


def _gpu_config(num_blocks=8, block_size=2):
    """A config that claims a GPU device: validation runs before any GPU call."""

    return SimpleNamespace(num_blocks=num_blocks, block_size=block_size, device=torch.device("cuda", 0),
                           dtype=torch.bfloat16)


def test_bound_classes_are_what_the_package_exports(host_classes) -> None:
    assert lv.KVCacheError is HostKVCacheError and errors.KVCacheError is HostKVCacheError
    assert lv.KVCacheCapacityError is HostCapacityError
    assert lv.ExecutionError is HostExecutionError and lv.ExecutionNotReadyError is HostNotReadyError


def test_metadata_and_plan_sites_raise_the_host_class(host_classes) -> None:
    md = _metadata(tables=((0, 9),))
    with pytest.raises(HostKVCacheError, match="out-of-range"):
        md.validate_block_tables(num_blocks=8, block_size=2)
    with pytest.raises(HostKVCacheError, match="out-of-range"):
        StepPlan(md, block_size=2, device=CPU, num_blocks=8)
    with pytest.raises(HostKVCacheError, match="out-of-range"):
        facts_of(md).check_tables(num_blocks=8, block_size=2)
    with pytest.raises(HostKVCacheError, match="does not cover"):
        _metadata(tables=((0,),)).slot_mapping(block_size=2, device=CPU)
    # A foreign metadata object (light-vllm's class) goes through the same rules.
    foreign = SimpleNamespace(block_tables=((0, 1), (1, 2)), num_computed_tokens=(3, 3),
                              query_layouts=(lv.linear_query_layout(1),) * 2, num_reserved_query_tokens=(1, 1),
                              num_readonly_prefix_blocks=(0, 0))
    with pytest.raises(HostKVCacheError, match="across requests"):
        StepPlan(foreign, block_size=2, device=CPU, num_blocks=8)


def test_cache_and_copy_sites_raise_the_host_class(host_classes) -> None:
    spec = lv.ModelKVCacheSpec((lv.AttentionLayerSpec("l0", 4, 2, 64),))
    with pytest.raises(HostKVCacheError, match="requires a GPU"):
        PagedKVCache(spec, lv.PagedKVCacheConfig(num_blocks=4, block_size=2))
    with pytest.raises(HostKVCacheError, match="float32, float16 and bfloat16"):
        dtype_code(torch.int8)
    gpu_cache = SimpleNamespace(config=_gpu_config())
    kw = dict(num_computed_tokens=1, num_query_tokens=2, num_reserved_query_tokens=2, retained_query_indices=(1,))
    with pytest.raises(HostKVCacheError, match="invalid physical block"):
        hip_compact(gpu_cache, (0, 99), **kw)
    with pytest.raises(HostKVCacheError, match="same slot"):
        _compact_plan(gpu_cache.config, [dict(block_ids=(0, 1), **kw)] * 2)
    with pytest.raises(HostKVCacheError, match="disjoint"):
        hip_block_copy(gpu_cache, (1, 2), (2, 3))
    cpu_cache = SimpleNamespace(config=lv.PagedKVCacheConfig(num_blocks=4, block_size=2))
    with pytest.raises(HostKVCacheError, match="requires a GPU"):
        hip_block_copy(cpu_cache, (1,), (2,))
    # A cache object without the layer: write_prepared's and layer_spec's lookups.
    cache = PagedKVCache.__new__(PagedKVCache)
    cache._layers, cache._layer_specs = {}, {}
    with pytest.raises(HostKVCacheError, match="was not found"):
        cache.layer_spec("missing")
    with pytest.raises(HostKVCacheError, match="was not found"):
        cache.write_prepared("missing", torch.zeros(1, 2, 64), torch.zeros(1, 2, 64), None)


def test_backend_sites_raise_the_host_class(host_classes) -> None:
    cpu_cache = SimpleNamespace(config=lv.PagedKVCacheConfig(num_blocks=4, block_size=2))
    with pytest.raises(HostKVCacheError, match="requires a GPU"):
        lv.HipPagedAttentionBackend().create(cpu_cache, _metadata())
    spec = lv.AttentionLayerSpec("l0", 4, 2, 64)
    cache = SimpleNamespace(config=lv.PagedKVCacheConfig(num_blocks=4, block_size=2),
                            layer_spec=lambda layer_id: spec)
    ctx = HipPagedAttention.__new__(HipPagedAttention)
    ctx._cache, ctx._config, ctx._layer_ids, ctx._statics = cache, cache.config, set(), {}
    ctx._plan = SimpleNamespace(num_query_tokens=1)
    q, kv = torch.zeros(1, 4, 64), torch.zeros(1, 2, 64)
    with pytest.raises(HostKVCacheError, match="three dimensions"):
        ctx.forward("l0", q[0], kv, kv, scale=1.0)
    with pytest.raises(HostKVCacheError, match="ran more than once"):
        ctx.forward("l0", q, kv, kv, scale=1.0)
    ctx._layer_ids = set()
    with pytest.raises(HostKVCacheError, match="token count"):
        ctx.forward("l0", torch.zeros(2, 4, 64), torch.zeros(2, 2, 64), torch.zeros(2, 2, 64), scale=1.0)
    ctx._layer_ids = set()
    with pytest.raises(HostKVCacheError, match="dtype and device"):
        ctx.forward("l0", q.double(), kv, kv, scale=1.0)


def test_native_sites_raise_the_host_classes(host_classes, monkeypatch) -> None:
    with pytest.raises(HostExecutionError, match="lvamd_x failed"):
        native.check(-1, "lvamd_x")
    missing = Path("/nonexistent/liblvamd_hip.so")
    native.load.cache_clear()
    monkeypatch.setattr(native, "library_path", lambda: missing)
    try:
        with pytest.raises(HostNotReadyError, match="not built"):
            native.load()
        with pytest.raises(HostNotReadyError):
            lv.HipPagedAttentionBackend()
    finally:
        monkeypatch.undo()
        native.load.cache_clear()
    native.host.cache_clear()
    monkeypatch.setattr(native, "host_path", lambda: Path("/nonexistent/_lvamd_host.so"))
    try:
        with pytest.raises(HostNotReadyError, match="host planner"):
            native.host()
    finally:
        monkeypatch.undo()
        native.host.cache_clear()


def test_a_light_vllm_style_handler_turns_compact_errors_into_execution_errors(host_classes) -> None:
    """The shape of PagedStepHandler.compact (worker.py:306-323) with the bound
    classes: the backend's compact failure is caught and re-raised as the
    host's ExecutionError carrying the message."""

    gpu_cache = SimpleNamespace(config=_gpu_config())

    def handler_compact():
        try:
            return hip_compact(gpu_cache, (0, 1, 2), num_computed_tokens=1, num_query_tokens=2,
                               num_reserved_query_tokens=2, retained_query_indices=(1,))
        except lv.KVCacheError as exc:
            raise lv.ExecutionError(str(exc)) from exc

    with pytest.raises(HostExecutionError, match="exactly cover"):
        handler_compact()


def test_bind_checks_the_hierarchy_and_restores() -> None:
    with pytest.raises(TypeError, match="derive"):
        errors.bind(kv_cache_error=HostKVCacheError, kv_cache_capacity_error=RuntimeError)
    with pytest.raises(TypeError, match="exception class"):
        errors.bind(execution_error=42)
    errors.bind(kv_cache_error=HostKVCacheError)
    try:
        assert issubclass(lv.KVCacheCapacityError, HostKVCacheError)
        assert lv.ExecutionError is not HostExecutionError
    finally:
        errors.bind()
    assert lv.KVCacheError is not HostKVCacheError
    assert lv.KVCacheError.__name__ == "KVCacheError" and issubclass(lv.ExecutionNotReadyError, lv.ExecutionError)


def test_no_raise_site_bypasses_the_binding() -> None:
    """Every module raises through ``errors.<Name>`` (looked up at raise time);
    none imports the classes by name or defines its own."""

    names = "KVCacheError|KVCacheCapacityError|ExecutionError|ExecutionNotReadyError"
    for path in sorted(PACKAGE.glob("*.py")):
        text = path.read_text()
        assert not re.search(rf"raise ({names})\(", text), f"{path.name} raises an unbound class"
        assert not re.search(rf"from light_vllm_amd\.errors import .*({names})", text), path.name
        if path.name != "errors.py":
            assert not re.search(rf"class ({names})\b", text), path.name


def test_light_vllm_classes_are_bound_when_importable(tmp_path) -> None:
    """With light-vllm's modules importable, the package raises their classes
    without any call to ``bind`` (a stand-in light_vllm package here)."""

    pkg = tmp_path / "light_vllm" / "runtime" / "execution"
    pkg.mkdir(parents=True)
    for d in (tmp_path / "light_vllm", tmp_path / "light_vllm" / "runtime", pkg):
        (d / "__init__.py").write_text("")
    (tmp_path / "light_vllm" / "runtime" / "kv_cache.py").write_text(
        "class KVCacheError(RuntimeError): pass\nclass KVCacheCapacityError(KVCacheError): pass\n")
    (pkg / "interfaces.py").write_text(
        "class ExecutionError(RuntimeError): pass\nclass ExecutionNotReadyError(ExecutionError): pass\n")
    script = textwrap.dedent(f"""
        import importlib, sys
        sys.path[:0] = [{str(tmp_path)!r}, {str(PACKAGE.parent)!r}]
        importlib.import_module("light-vllm_amd")
        import light_vllm_amd as lv
        from light_vllm.runtime.kv_cache import KVCacheError
        from light_vllm.runtime.execution.interfaces import ExecutionError
        assert lv.KVCacheError is KVCacheError and lv.ExecutionError is ExecutionError
        try:
            lv.PagedAttentionMetadata(block_tables=((0, 9),), num_computed_tokens=(3,),
                query_layouts=(lv.linear_query_layout(1),)).validate_block_tables(num_blocks=8, block_size=2)
        except KVCacheError as exc:
            print("host class:", exc)
    """)
    out = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert "host class: block table contains an out-of-range physical block" in out.stdout


def test_every_import_path_reaches_the_same_modules() -> None:
    """``import light_vllm_amd.errors``, ``from light_vllm_amd import errors``
    and the directory's own name give one module object each, so a binding
    made through any of them is the one raise sites use (fresh interpreter:
    nothing imported before the package)."""

    script = textwrap.dedent(f"""
        import importlib, sys
        sys.path.insert(0, {str(PACKAGE.parent)!r})
        importlib.import_module("light-vllm_amd")
        import light_vllm_amd.errors as by_alias
        import light_vllm_amd.native as native_alias
        from light_vllm_amd import errors as by_attribute
        import light_vllm_amd as lv
        names = ("errors", "native", "facts", "plan", "backend", "metadata", "paged_cache", "interfaces", "layout")
        for name in names:
            assert sys.modules["light_vllm_amd." + name] is sys.modules["light-vllm_amd." + name], name
        assert by_alias is by_attribute is lv.errors and native_alias is lv.native
        class Host(RuntimeError):
            pass
        from light_vllm_amd.errors import bind
        bind(kv_cache_error=Host)
        try:
            lv.PagedAttentionMetadata(block_tables=((0, 9),), num_computed_tokens=(3,),
                query_layouts=(lv.linear_query_layout(1),)).validate_block_tables(num_blocks=8, block_size=2)
        except Host as exc:
            print("bound class:", exc)
    """)
    out = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    assert "bound class: block table contains an out-of-range physical block" in out.stdout
