"""Stream discipline of the Python host layer.

Every wrapper that launches on a caller-chosen stream makes that stream current while it
allocates its temporaries (outputs, workspaces), so torch's caching allocator ties the memory to
the stream the kernels run on; persistent workspaces are recorded on each stream that uses them.
"""
import inspect

import numpy as np
import pytest
import torch

from helixml_amd import lm, ssm

# functions that take a `stream` but only pass it on, or manage their own streams
_EXEMPT = {"_stream", "_torch_stream", "keep_for_stream", "_head", "decode_graph"}


def _stream_takers():
    for mod in (ssm, lm):
        for name, obj in vars(mod).items():
            if inspect.isfunction(obj) and obj.__module__ == mod.__name__:
                yield f"{mod.__name__}.{name}", obj
            elif inspect.isclass(obj) and obj.__module__ == mod.__name__:
                for mname, m in vars(obj).items():
                    if inspect.isfunction(m):
                        yield f"{mod.__name__}.{name}.{mname}", m


def test_every_launching_wrapper_allocates_on_its_launch_stream():
    """CPU check: each function or method with a ``stream`` parameter is wrapped by
    on_launch_stream (or is one of the listed helpers)."""
    missing, seen = [], 0
    for qual, fn in _stream_takers():
        short = qual.rsplit(".", 1)[-1]
        target = getattr(fn, "__wrapped__", fn)
        if "stream" not in inspect.signature(target).parameters or short in _EXEMPT:
            continue
        seen += 1
        if not getattr(fn, "on_launch_stream", False):
            missing.append(qual)
    assert seen >= 12, seen
    assert not missing, f"launching on a caller stream without allocating there: {missing}"


@pytest.mark.gpu
def test_temporaries_belong_to_the_launch_stream(dev, monkeypatch):
    """A segmented scan (it needs a workspace) launched on a side stream allocates its output,
    final state and workspace while that stream is current, and computes what the default-stream
    call computes."""
    from tests.util import scan_inputs
    x = scan_inputs(1, 4096, 64, 16, seed=7)
    d = {k: (None if v is None else torch.from_numpy(v).to(dev)) for k, v in x.items()}
    assert ssm.selective_scan_workspace_size(1, 4096, 64, 16) > 0
    ref, ref_last = ssm.selective_scan_fwd(**d, return_last_state=True)
    torch.cuda.synchronize()

    seen = []

    def spy(fn):
        def alloc(*a, **k):
            seen.append(torch.cuda.current_stream())
            return fn(*a, **k)
        return alloc

    monkeypatch.setattr(ssm.torch, "empty", spy(torch.empty))
    monkeypatch.setattr(ssm.torch, "empty_like", spy(torch.empty_like))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    out, last = ssm.selective_scan_fwd(**d, return_last_state=True, stream=side)
    monkeypatch.undo()
    torch.cuda.synchronize()
    # out (empty_like), last and the workspace (empty)
    assert len(seen) == 3 and all(s == side for s in seen), seen
    assert torch.equal(out, ref) and torch.equal(last, ref_last)
    # a raw handle works the same way
    out2 = ssm.selective_scan_fwd(**d, stream=side.cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out2, ref)
    assert np.isfinite(out.cpu().numpy()).all()
