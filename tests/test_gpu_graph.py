"""launchSpmmInt8 and launchSpmmInt8NoAlloc captured into a HIP graph (torch.cuda.CUDAGraph) and
replayed. Neither records an allocation or a memset: the completion counters return to zero by
themselves, and the no-alloc entry point clears its scratch counters with a kernel. Each replay must
therefore give the eager result bit for bit. c2's plan has split SWs, so every replay runs the
tickets and the merge; eager launches and synchronisations run between the replays."""
import pytest

import tcc_spmm_amd as T
from gpu_cases import features, gpu_prepare

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("entry", ["workspace", "noalloc"])
@pytest.mark.parametrize("feats,waves", [(128, "1"), (128, "2"), (256, "1")])
def test_spmm_replays_from_a_hip_graph(gpu, entry, feats, waves, launch_overrides):
    import torch
    from tcc_spmm_amd.device import TorchDeviceMatrix, launch_spmm_int8_noalloc
    launch_overrides(task_waves=int(waves))
    print(f"graph case: {entry} F{feats} waves {waves}", flush=True)
    csr = T.synth_csr("c2")
    fmt = T.convert_csr_to_sw32(csr.rows, csr.cols, csr)
    assert fmt.partial_count > 0
    packed, scale, *_ = gpu_prepare(features(csr.cols, feats, seed=55), gpu)
    dm = TorchDeviceMatrix(fmt, feats, device=gpu)

    def launch(y):
        if entry == "workspace":
            dm.spmm(packed, scale, y)
        else:
            launch_spmm_int8_noalloc(dm.view, packed, scale, y, csr.rows, csr.cols, feats,
                                     fmt.partial_count)

    want = torch.empty((csr.rows, feats), device=gpu)
    launch(want)
    torch.cuda.synchronize()
    y = torch.full_like(want, float("nan"))
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up off the default stream, as capture expects
        launch(y)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch(y)
    other = torch.empty_like(want)
    for i in range(4):
        y.fill_(float("nan"))
        launch(other)  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), want.view(torch.int32)), f"replay {i}"
        assert torch.equal(other.view(torch.int32), want.view(torch.int32)), f"eager {i}"
        if entry == "workspace":
            assert int(dm.counters.abs().sum()) == 0, f"counters after replay {i}"
