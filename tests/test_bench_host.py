"""Host-side checks of bench.py's launchers (no GPU).

bench.py times the kernels through pre-marshalled launchers that hand raw
device addresses to the C ABI.  A launcher that kept only the address of a
tensor and not the tensor lets the allocator hand that memory to a later
allocation, after which a launch reads or writes someone else's data.  These
tests pin that every address a launcher passes belongs to a tensor the
launcher itself holds, and that bench.py makes no C-ABI call or address
conversion outside that one launcher factory.
"""
import ast
import ctypes
import gc
import os
import weakref

import torch

import bench

BENCH_PY = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "bench.py")


def test_lean_launch_holds_every_tensor_it_points_at():
    calls = []

    def fake_entry(*args):
        calls.append(args)
        return 0

    a = torch.arange(64, dtype=torch.float32)
    b = torch.zeros(5, dtype=torch.int32)
    stream = 0x7F00_0000_1000  # a raw pointer-sized int, passed through as an address
    refs = [weakref.ref(a), weakref.ref(b)]
    ptrs = (a.data_ptr(), b.data_ptr())
    run = bench.lean_launch(fake_entry, a, 7, 1.5, b, stream)
    del a, b
    gc.collect()
    # the launcher is the only owner left, and it still holds both tensors
    assert all(r() is not None for r in refs)
    assert tuple(t.data_ptr() for t in run.keep) == ptrs
    # every address argument is a kept tensor's, or the stream
    addr = [x.value for x in run.args if isinstance(x, ctypes.c_void_p)]
    assert addr == [ptrs[0], ptrs[1], stream]
    assert run.args[1] == 7 and run.args[2] == 1.5
    run()
    run()
    assert len(calls) == 2 and calls[0] == run.args
    assert run.status == [0, 0]
    bench.check_lean(run)
    assert run.status == []
    # dropping the launcher releases the tensors
    del run
    gc.collect()
    assert all(r() is None for r in refs)


def test_bench_calls_the_c_abi_only_through_lean_launch():
    tree = ast.parse(open(BENCH_PY).read())
    lean = next(n for n in tree.body if isinstance(n, ast.FunctionDef) and n.name == "lean_launch")
    inside = {id(n) for n in ast.walk(lean)}
    for node in ast.walk(tree):
        if isinstance(node, ast.Call) and isinstance(node.func, ast.Attribute):
            # a direct call of an ftq_* entry point would bypass the launcher
            assert not node.func.attr.startswith("ftq_") or node.func.attr in (
                "ftq_paged_choose_splits", "ftq_v1_default_splits", "ftq_paged_default_splits",
                "ftq_v1_workspace_bytes", "ftq_paged_workspace_bytes", "ftq_v1_slot_bytes",
                "ftq_codebook_class"), f"bench.py:{node.lineno} calls {node.func.attr} directly"
            if node.func.attr == "data_ptr":
                assert id(node) in inside, f"bench.py:{node.lineno} takes a raw address outside lean_launch"
