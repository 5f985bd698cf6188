"""Graph-captured multi-tick rollout == eager native ticks, bitwise (MI355X)."""

from __future__ import annotations

import pytest
import torch

from cases import column_drive, make_case
from neurosim_gpu import MatrixRollout, NativeDendriticMatrixRuntime

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("batch,fmt", [(1, None), (8, None), (1, "fp8"), (3, "nvfp4")])
def test_graph_rollout_matches_eager(gpu, batch, fmt):
    case = make_case(4000, 80_000, 2, gpu)
    drive = column_drive(batch).to(gpu)
    kwargs = {} if fmt is None else {"weight_format": fmt}
    eager = NativeDendriticMatrixRuntime(case.topology, case.model,
                                         torch.zeros(batch, 4000, device=gpu), **kwargs)
    seeded = NativeDendriticMatrixRuntime(case.topology, case.model,
                                          torch.zeros(batch, 4000, device=gpu), **kwargs)
    for _ in range(3):            # non-trivial starting states
        eager.step(drive, dendritic_drive=0.1)
        seeded.step(drive, dendritic_drive=0.1)
    rollout = MatrixRollout(seeded, 16, drive=drive, dendritic_drive=0.1)
    for replay in range(3):
        rollout.run()
        # eager work between replays, then compare every replay
        for _ in range(16):
            eager.step(drive, dendritic_drive=0.1)
        torch.cuda.synchronize()
        for field in ("state", "dendritic_state", "adaptation_state"):
            assert torch.equal(getattr(rollout, field), getattr(eager, field)), (replay, field)
    rollout.write_back()
    seeded.step(drive, dendritic_drive=0.1)
    eager.step(drive, dendritic_drive=0.1)
    assert torch.equal(seeded.state, eager.state)


def test_rollout_rejects_odd_ticks(gpu):
    case = make_case(100, 1000, 2, gpu)
    runtime = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(1, 100, device=gpu))
    with pytest.raises(ValueError, match="even"):
        MatrixRollout(runtime, 3)
