"""Helpers for GPU parity tests: run one plan over numpy data via torch buffers."""
import numpy as np

import cubutterfly_amd as cb

_TORCH_DTYPES = None


def _torch_dtype(torch, np_dtype):
    table = {np.dtype(np.float32): torch.float32, np.dtype(np.float16): torch.float16,
             np.dtype(np.uint32): torch.int32, np.dtype(np.uint64): torch.int64,
             np.dtype(np.complex64): torch.complex64}
    return table[np.dtype(np_dtype)]


def to_device(torch, array):
    a = np.ascontiguousarray(array)
    view = a.view(np.int32) if a.dtype == np.uint32 else a.view(np.int64) if a.dtype == np.uint64 else a
    return torch.from_numpy(view.copy()).to("cuda")


def to_host(torch, tensor, np_dtype):
    out = tensor.cpu().numpy()
    return out.view(np_dtype)


def run_plan(torch, lib, transform, host_input, stream, in_place=False, **plan_args):
    """Execute `transform` on host_input through the C ABI; returns the host result."""
    x = to_device(torch, host_input)
    with cb.Plan(lib, transform, stream=stream, **plan_args) as plan:
        assert plan.input_size() == x.numel() * x.element_size()
        # Output shaped like the input when the sizes agree, else flat (the
        # zero-extended embedding changes the extents).
        out_elems = plan.output_size() // x.element_size()
        if in_place:
            y = x
        elif out_elems == x.numel():
            y = torch.empty_like(x)
        else:
            y = torch.empty(out_elems, dtype=x.dtype, device="cuda")
        ws_bytes = plan.workspace_size()
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda") if ws_bytes else None
        if ws is not None:
            plan.set_workspace(ws, ws_bytes)
        plan.execute(x, y)
        torch.cuda.synchronize()
    return to_host(torch, y, np.dtype(host_input.dtype))
