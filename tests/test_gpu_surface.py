"""The intent.jit call surface on the GPU: run, explicit outputs, prepare/launch/result,
streams, observation, as_torch_op (with torch.compile-style fake tensors) and errors."""
import numpy as np
import pytest
import torch

import intent_amd as intent
import oracle
from intent_amd.examples import inputs
from intent_amd.examples.kernels.backward.softmax import softmax_backward_f16
from intent_amd.examples.kernels.normalization.softmax import stable_softmax, stable_softmax_f16
from intent_amd.runtime.hip.library import LIBRARY_PATH
from tests.gpu_util import announce, assert_f32_rel

pytestmark = pytest.mark.gpu


def test_native_library_is_the_one_loaded(device):
    announce("library loaded")
    intent.jit(stable_softmax, backend="hip").run(torch.zeros(2, 8, device=device))
    maps = open("/proc/self/maps").read()
    assert str(LIBRARY_PATH) in maps


def test_run_prepare_launch_result(device):
    announce("prepare/launch/result")
    x = torch.from_numpy(inputs.normal(np.random.default_rng(0), (64, 256), "f32", 4)).to(device)
    kernel = intent.jit(stable_softmax, backend="hip")
    call = kernel.prepare(x)
    y = call.result()                                     # allocated at prepare, no launch yet
    assert y.shape == x.shape
    call.launch()
    torch.cuda.synchronize()
    want = oracle.softmax_fwd(x.cpu().numpy())
    assert_f32_rel(y.cpu().numpy(), want)
    x.mul_(0.5)                                           # relaunch sees the new contents
    call.launch()
    assert_f32_rel(call.result().cpu().numpy(), oracle.softmax_fwd(x.cpu().numpy()))
    obs = call.observation
    assert obs.provider == "hip" and obs.entry == "intent_hip_softmax_fwd" and obs.kernel
    assert kernel.interface.parameters[0].name == "x"
    assert len(call.inspect_configurations()) == 1
    assert kernel.artifacts[0].observation is not None
    artifact = kernel.artifacts[0]
    assert "stable_softmax" in artifact.source and "intent_hip_softmax_fwd" in artifact.source
    assert artifact.ir["intent"] and "no KIR stage" in artifact.mlir
    explicit = torch.empty_like(x)
    assert kernel(x, explicit) is None
    assert_f32_rel(explicit.cpu().numpy(), oracle.softmax_fwd(x.cpu().numpy()))
    artifact = kernel.artifacts[0]
    other = torch.empty_like(x)
    artifact.launch(x, other)
    assert torch.equal(other, explicit)


def test_launches_follow_the_current_stream(device):
    announce("streams")
    x = torch.from_numpy(inputs.normal(np.random.default_rng(1), (512, 1024), "f16", 3)).to(device)
    kernel = intent.jit(stable_softmax_f16, backend="hip")
    reference = kernel.run(x)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        out = kernel.run(x)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert torch.equal(out, reference)


def test_graph_capture_replays(device):
    announce("hip graph capture")
    x = torch.from_numpy(inputs.normal(np.random.default_rng(2), (256, 2048), "f16", 3)).to(device)
    dy = torch.from_numpy(inputs.normal(np.random.default_rng(3), (256, 2048), "f16")).to(device)
    fwd = intent.jit(stable_softmax_f16, backend="hip").prepare(x)
    bwd = intent.jit(softmax_backward_f16, backend="hip").prepare(fwd.result(), dy)
    fwd.launch()
    bwd.launch()
    torch.cuda.synchronize()
    eager_y, eager_dx = fwd.result().clone(), bwd.result().clone()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            fwd.launch()
            bwd.launch()
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        fwd.result().zero_()
        bwd.result().zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(fwd.result(), eager_y) and torch.equal(bwd.result(), eager_dx)


def test_as_torch_op_and_fake_tensors(device):
    announce("as_torch_op")
    x = torch.from_numpy(inputs.normal(np.random.default_rng(4), (32, 128), "f32", 4)).to(device)
    kernel = intent.jit(stable_softmax, backend="hip")
    kernel.prepare(x)
    op = kernel.as_torch_op("intent_amd_test::stable_softmax")
    y = op(x)
    assert_f32_rel(y.cpu().numpy(), oracle.softmax_fwd(x.cpu().numpy()))
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode() as mode:
        fake = mode.from_tensor(x)
        out = op(fake)
        assert out.shape == x.shape and out.dtype == torch.float32

    compiled = torch.compile(lambda t: op(t) * 2.0, backend="eager")
    assert torch.allclose(compiled(x), y * 2.0)


def test_errors_on_gpu(device):
    announce("errors")
    kernel = intent.jit(stable_softmax, backend="hip")
    with pytest.raises(TypeError):
        kernel.run(torch.zeros(2, 2, device=device, dtype=torch.float16))
    with pytest.raises(ValueError):
        kernel.run(torch.zeros(2, device=device))
    with pytest.raises(ValueError):
        kernel.run(torch.zeros(2, 2))                     # CPU tensor
    with pytest.raises(intent.CompilationStageError):
        intent.jit(stable_softmax, backend="hip", constexprs={"BOGUS": 1}).run(torch.zeros(2, 2, device=device))


def test_saved_program_runs_like_jit(device, tmp_path):
    """examples/softmax.py --program: a generated program saved, loaded and bound to a local target
    runs the same kernel as intent.jit."""
    announce("saved program")
    from intent_amd.examples.kernels.normalization.softmax import stable_softmax_f16
    from intent_amd.targets.hip import HipTarget
    from intent_amd.targets.local import resolve_local, select_device

    x = torch.randn((512, 1000), device=device, dtype=torch.float16)
    path = intent.generate(stable_softmax_f16, target=HipTarget(device.index or 0)).save(tmp_path / "softmax")
    target = resolve_local("hip", select_device("hip", (x,), str(device)))
    softmax = intent.GeneratedProgram.load(path).materialize(target=target)
    y = softmax.run(x)
    want = intent.jit(stable_softmax_f16, backend="hip").run(x)
    assert torch.equal(y, want)
    out = torch.empty_like(x)
    call = softmax.prepare(x, outputs=(out,))
    call.launch()
    assert call.result() is out and torch.equal(out, want)


def test_static_workspace_refuses_staging(device):
    """With backend_options={"workspace": "static"} the provider allocates nothing at prepare, so a
    view the kernel cannot read in place (here a vector of stride 2) is refused instead of staged
    through a copy, as the default policy does."""
    announce("workspace=static staging")
    from intent_amd.examples.kernels.sparse.csr_spmv import csr_spmv

    offsets = torch.tensor([0, 2, 3, 3, 5], dtype=torch.int32, device=device)
    columns = torch.tensor([0, 3, 1, 2, 3], dtype=torch.int32, device=device)
    values = torch.tensor([1.0, 2.0, 3.0, 4.0, 5.0], device=device)
    strided = torch.arange(8.0, device=device)[::2]                      # x = [0, 2, 4, 6]
    with pytest.raises(ValueError):
        intent.jit(csr_spmv, backend="hip", backend_options={"workspace": "static"}).run(
            offsets, columns, values, strided)
    y = intent.jit(csr_spmv, backend="hip").run(offsets, columns, values, strided)
    assert y.cpu().tolist() == [12.0, 6.0, 0.0, 46.0]
    with pytest.raises(ValueError):
        intent.jit(csr_spmv, backend="hip", backend_options={"workspace": "pinned"}).run(
            offsets, columns, values, strided.contiguous())
