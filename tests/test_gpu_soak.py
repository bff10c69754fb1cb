"""Bitwise soak of the register-resident softmax on C5 (4,194,304 rows of
bf16 D=128, long-tail segments up to 200,000 rows): 100 classified calls on
one workspace, each compared bit for bit with the first, stopping at the
first mismatch.

Between calls everything the workspace contract does not keep is filled with
garbage: every byte outside the counters and the statistics arena, and the
arena's byte ranges the last call recorded as published (the pairs and group
rows its merges folded), which the next call's classification must zero
before its merges poll them -- a pair left over from the previous call, or
one folded before its publication is visible, would change the output. Every
tenth call the whole arena is filled and recorded as unknown (slot 12 = 1),
as another plan's buffers would leave it.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import native  # noqa: E402
from ragged.workloads import CONFIGS  # noqa: E402

DEVICE = torch.device("cuda", 0)
ARENA = ("pairs", "final_pairs", "arrive", "deferred")
CLEAN_SLOT, DIRTY_SLOT, DIRTY_RANGES = 12, 14, 3
CALLS = 100


def test_c5_classified_soak_bitwise():
    w = CONFIGS["c5"](711)
    spec = native.make_spec("softmax", "bf16", w.offsets_dtype, w.d)
    assert native.uses_fused(spec)
    module = native.NativeModule(0, spec)
    x = torch.from_numpy(w.values).to(DEVICE).to(torch.bfloat16).contiguous()
    off = torch.from_numpy(w.offsets).to(DEVICE)
    n, b = x.shape[0], len(w.offsets) - 1
    plan = module.plan(n, b, "classified")
    names = [native.ROLES[plan.roles[i]] for i in range(plan.launches)]
    assert names == ["classify", "fused"], names
    spans = {name: (offset, nbytes) for name, offset, nbytes in plan.buffers}
    counters = spans["class_counts"]
    arena = (min(spans[k][0] for k in ARENA), max(spans[k][0] + spans[k][1] for k in ARENA))
    arena = (arena[0], (arena[1] + 255) // 256 * 256)
    workspace = torch.zeros((int(plan.workspace_bytes),), dtype=torch.uint8, device=DEVICE)
    first = torch.empty_like(x)
    out = torch.empty_like(x)
    stream = torch.cuda.current_stream().cuda_stream

    def call(target):
        module.run(plan, x.data_ptr(), off.data_ptr(), target.data_ptr(), None, workspace.data_ptr(),
                   int(plan.workspace_bytes), stream)

    call(first)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(first.float()).all())
    for i in range(1, CALLS):
        slots = workspace[counters[0]:counters[0] + counters[1]].view(torch.int64)
        record = slots[:DIRTY_SLOT + 2 * DIRTY_RANGES].cpu().numpy()
        assert record[CLEAN_SLOT] == arena[1] - arena[0] + 2
        workspace[arena[1]:].fill_(0xA5)
        if i % 10 == 0:
            workspace[arena[0]:arena[1]].fill_(0xA5)
            slots[CLEAN_SLOT] = 1
        else:
            for r in range(DIRTY_RANGES):
                lo, hi = int(record[DIRTY_SLOT + 2 * r]), int(record[DIRTY_SLOT + 2 * r + 1])
                workspace[arena[0] + lo:arena[0] + hi].fill_(0xA5)
        out.fill_(float("nan"))
        call(out)
        torch.cuda.synchronize()
        same = torch.equal(out.view(torch.int16), first.view(torch.int16))
        if not same:
            rows = torch.nonzero((out.view(torch.int16) != first.view(torch.int16)).any(dim=1)).flatten()
            segment = int(np.searchsorted(w.offsets, int(rows[0]), side="right") - 1)
            pytest.fail(f"call {i}: {rows.numel()} rows differ from the first call's, first row {int(rows[0])} "
                        f"(segment {segment}, {int(w.lengths[segment])} rows)")
    print(f"{CALLS} classified C5 calls bit-identical")
    module.close()
