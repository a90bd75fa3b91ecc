"""The allocation-free scheduled attention (tjk_flash_fwd_sched_static),
called through the C-ABI, against the workspace-taking entry point it
shares its kernel with: bitwise-equal outputs on two calls in a row, the
second with a smaller input, with key-split items so the static partials and
flags are used.  (The rejection of a work list needing more slots than the
static array holds makes no HIP call and is tested on the CPU, in
test_host.py.)"""

import ctypes

import pytest
import torch

from tjkernels import _lib, schedule as sched_mod

pytestmark = pytest.mark.gpu


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _case(device, lengths, heads, hd, dt, seed):
    t = sum(lengths)
    g = torch.Generator()
    g.manual_seed(seed)
    qkv = torch.randn(t, 3, heads, hd, generator=g).to(dt).to(device)
    cu = [0]
    for n in lengths:
        cu.append(cu[-1] + n)
    cu_d = torch.tensor(cu, dtype=torch.int32, device=device)
    sched = sched_mod.build_schedule(lengths, heads, hd, True, dt, device, slots=100000, min_split=2,
                                     split_factor=1.0)
    assert sched.n_slots > 0
    return qkv, cu_d, sched


def _run(lib, fn, qkv, cu_d, sched, lengths, heads, hd, dt, static):
    t = qkv.shape[0]
    out = torch.full((t, heads * hd), 7.0, dtype=dt, device=qkv.device)
    ss, sc, sh, _ = qkv.stride()
    args = [qkv.data_ptr(), ss, sc, sh, out.data_ptr(), out.stride(0), len(lengths), max(lengths), heads, hd,
            hd ** -0.5, 1, cu_d.data_ptr(), sched.work.data_ptr(), sched.work.shape[0],
            sched.n_lists or sched.work.shape[0]]
    if static:
        rc = lib.tjk_flash_fwd_sched_static(*args, sched.n_slots, _lib.DTYPE_CODES[dt], _stream())
    else:
        rc = lib.tjk_flash_fwd_sched(*args, sched.partials.data_ptr(),
                                     sched.partials.numel() * sched.partials.element_size(), sched.n_slots,
                                     _lib.DTYPE_CODES[dt], _stream())
    assert rc == 0, lib.tjk_last_error_string()
    return out


@pytest.mark.parametrize("dt,hd", [(torch.bfloat16, 64), (torch.float16, 128)])
def test_static_workspace_matches_workspace_entry(device, dt, hd):
    lib = _lib.load()
    heads = 3
    for lengths, seed in (([300, 0, 129, 700, 64], 1), ([200, 5], 2)):  # the second call is smaller
        qkv, cu_d, sched = _case(device, lengths, heads, hd, dt, seed)
        want = _run(lib, lib.tjk_flash_fwd_sched, qkv, cu_d, sched, lengths, heads, hd, dt, static=False)
        got = _run(lib, lib.tjk_flash_fwd_sched_static, qkv, cu_d, sched, lengths, heads, hd, dt, static=True)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"static-workspace output differs for lengths {lengths}"
        assert torch.isfinite(got.float()).all()
        assert sched_mod.error_count(sched) == 0

