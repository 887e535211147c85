"""Inverse-rendering samples of mlx-swift-diffrast on the HIP path.

The reference validates its gradients end to end with three sample programs
(Sources/ColorFitExample, PoseFitExample and MeshFitExample, README.md:69-75).
This module holds their pieces, MI355X-native:

  * `mse_loss`: the samples' `lossFn`, `((out - target)^2).mean()`, as one
    kernel that also writes the gradient (dr_mse_loss);
  * `Adam`: the samples' optimizer (MLXDiffRastExamples/Adam.swift), one
    kernel per step (dr_adam_step);
  * the three scenes and their optimisation loops (`color_fit`, `pose_fit`,
    `mesh_fit`), with the reference's sizes, steps and learning rates.

The animated GIF output of the samples is not reproduced (macOS image I/O).
Run a sample with `python -m diffrast.fit color|pose|mesh`.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch

from . import _lib
from .ops import DiffRast
from .ops import _stream as _stream_handle


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream():
    return _stream_handle().value


# ---------------------------------------------------------------------------
# loss
# ---------------------------------------------------------------------------

class _MSEFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, out, target):
        lib = _lib.load()
        loss = torch.empty((), device=out.device, dtype=torch.float32)
        d_out = torch.empty_like(out) if ctx.needs_input_grad[0] else None
        _lib.check(lib.dr_mse_loss(_ptr(out), _ptr(target), out.numel(), _ptr(loss),
                                   _ptr(d_out), _stream()))
        ctx.save_for_backward(d_out)
        return loss

    @staticmethod
    def backward(ctx, g):
        (d_out,) = ctx.saved_tensors
        return d_out * g, None


def mse_loss(out: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """Mean of (out - target)^2 over every element (ColorFitExample/main.swift:62-66).
    Differentiable in `out`; the gradient is formed by the same kernel."""
    if tuple(out.shape) != tuple(target.shape):
        raise ValueError(f"mse_loss: shapes differ ({list(out.shape)} vs {list(target.shape)})")
    if not out.is_cuda or not target.is_cuda:
        raise ValueError("mse_loss: tensors must be on a ROCm device")
    if out.numel() == 0:
        raise ValueError("mse_loss: empty tensors")
    return _MSEFn.apply(out.to(torch.float32).contiguous(),
                        target.detach().to(torch.float32).contiguous())


# ---------------------------------------------------------------------------
# optimizer
# ---------------------------------------------------------------------------

class Adam:
    """Plain Adam for one parameter tensor (MLXDiffRastExamples/Adam.swift:8-44).
    The state (m, v, t) lives on the instance; `step` returns the updated
    parameter as a new tensor, like the reference."""

    def __init__(self, shape: Sequence[int], learningRate: float = 1e-2, beta1: float = 0.9,
                 beta2: float = 0.999, eps: float = 1e-8, device=None):
        self.learningRate = float(learningRate)
        self.beta1 = float(beta1)
        self.beta2 = float(beta2)
        self.eps = float(eps)
        dev = device if device is not None else torch.device("cuda", torch.cuda.current_device())
        self.m = torch.zeros(tuple(shape), device=dev, dtype=torch.float32)
        self.v = torch.zeros(tuple(shape), device=dev, dtype=torch.float32)
        self.t = 0

    def step(self, param: torch.Tensor, grad: torch.Tensor,
             mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Adam.swift:36-43.  `mask` multiplies the gradient first (the
        samples' posMask)."""
        if tuple(param.shape) != tuple(self.m.shape) or tuple(grad.shape) != tuple(self.m.shape):
            raise ValueError(f"Adam.step: param and grad must have shape {list(self.m.shape)}")
        if mask is not None and tuple(mask.shape) != tuple(self.m.shape):
            raise ValueError(f"Adam.step: mask must have shape {list(self.m.shape)}")
        lib = _lib.load()
        self.t += 1
        p = param.detach().to(torch.float32).contiguous()
        g = grad.detach().to(torch.float32).contiguous()
        mk = None if mask is None else mask.to(device=p.device, dtype=torch.float32).contiguous()
        out = torch.empty_like(p)
        _lib.check(lib.dr_adam_step(_ptr(p), _ptr(g), _ptr(mk), _ptr(self.m), _ptr(self.v),
                                    _ptr(out), p.numel(), self.t, self.learningRate, self.beta1,
                                    self.beta2, self.eps, _stream()))
        return out

    def step_(self, param: torch.Tensor, grad: torch.Tensor,
              mask: Optional[torch.Tensor] = None) -> None:
        """`step` written into `param` itself (contiguous float32 tensors of
        the state's shape, `mask` too): no allocation, one kernel."""
        for t in (param, grad) + (() if mask is None else (mask,)):
            if tuple(t.shape) != tuple(self.m.shape) or t.dtype != torch.float32 or \
                    not t.is_contiguous():
                raise ValueError(f"Adam.step_: tensors must be contiguous float32 "
                                 f"{list(self.m.shape)}")
        lib = _lib.load()
        self.t += 1
        _lib.check(lib.dr_adam_step(_ptr(param), _ptr(grad), _ptr(mask), _ptr(self.m),
                                    _ptr(self.v), _ptr(param), param.numel(), self.t,
                                    self.learningRate, self.beta1, self.beta2, self.eps,
                                    _stream()))


# ---------------------------------------------------------------------------
# the three samples
# ---------------------------------------------------------------------------

@dataclass
class FitResult:
    losses: List[float]        # loss before each step (what the samples print)
    param: torch.Tensor        # the optimised parameter
    target: torch.Tensor       # the parameter the target image was rendered from
    image_size: int


def _dev():
    if not torch.cuda.is_available():
        raise RuntimeError("the samples need a ROCm device")
    return torch.device("cuda", torch.cuda.current_device())


def _optimise(param, render, target_image, optimizer, steps, mask=None, log_every=0, log=None):
    """The samples' loop: value and gradient of the loss, then one Adam step.
    Losses stay on the device until the end (one read-back per logged step)."""
    losses = torch.empty(steps, device=param.device, dtype=torch.float32)
    for step in range(1, steps + 1):
        p = param.detach().requires_grad_(True)
        loss = mse_loss(render(p), target_image)
        (grad,) = torch.autograd.grad(loss, [p])
        losses[step - 1] = loss.detach()
        param = optimizer.step(p.detach(), grad, mask)
        if log is not None and log_every and (step % log_every == 0 or step == 1):
            log(f"  step {step:3d}  loss = {losses[step - 1].item():.6f}")
    return param, losses.cpu().tolist()


def _optimise_graph(param, render, target_image, optimizer, steps, mask=None, log_every=0,
                    log=None):
    """The same loop with the loss and its gradient captured once into a HIP
    graph and replayed each step: the parameter lives in one tensor that
    Adam updates in place, so a step costs a graph launch, a copy of the
    loss and the Adam kernel, not the host work of a dozen op calls.
    Warm-up and capture run on a stream of their own (the library sizes its
    per-stream scratch there before capture; nothing is allocated or waited
    for under capture), and so do the replays."""
    dev = param.device
    losses = torch.empty(steps, device=dev, dtype=torch.float32)
    mk = None if mask is None else mask.to(device=dev, dtype=torch.float32).contiguous()
    caller = torch.cuda.current_stream(dev)
    s = torch.cuda.Stream(dev)
    s.wait_stream(caller)
    with torch.cuda.stream(s):
        p = param.detach().to(torch.float32).contiguous().clone().requires_grad_(True)

        def loss_and_grad():
            loss = mse_loss(render(p), target_image)
            (grad,) = torch.autograd.grad(loss, [p])
            return loss, grad
        for _ in range(2):  # every call once on this stream before capture
            loss_and_grad()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            s_loss, s_grad = loss_and_grad()
        for step in range(1, steps + 1):
            graph.replay()
            losses[step - 1].copy_(s_loss)
            optimizer.step_(p.detach(), s_grad, mk)
            if log is not None and log_every and (step % log_every == 0 or step == 1):
                log(f"  step {step:3d}  loss = {losses[step - 1].item():.6f}")
        out = p.detach().clone()
    caller.wait_stream(s)
    return out, losses.cpu().tolist()


@dataclass
class Scene:
    """One sample's fixed data.  `kind` "color": the parameter is the vertex
    colours `attr` [1,V,3] of the fixed `pos`; "pose": the parameter is `pos`
    [1,V,4] (x, y optimised through `mask`) with fixed colours `attr`."""
    kind: str
    size: int
    tri: torch.Tensor
    pos: Optional[torch.Tensor]       # fixed positions ("color")
    attr: Optional[torch.Tensor]      # fixed colours ("pose")
    target: torch.Tensor              # parameter the target image is rendered from
    init: torch.Tensor                # initial parameter
    steps: int
    learning_rate: float
    mask: Optional[torch.Tensor] = None
    log_every: int = 20


def _f32(rows, dev, shape):
    return torch.tensor(rows, dtype=torch.float32, device=dev).view(*shape)


def color_scene(dev=None) -> Scene:
    """ColorFitExample/main.swift:22-80: one triangle, 64x64, target colours
    pure red / green / blue, start mid-grey, 120 steps at lr 0.05."""
    dev = dev or _dev()
    return Scene(
        kind="color", size=64,
        tri=torch.tensor([[0, 1, 2]], dtype=torch.int32, device=dev),
        pos=_f32([[-0.8, 0.8, 0, 1], [-0.8, -0.8, 0, 1], [0.8, 0.0, 0, 1]], dev, (1, 3, 4)),
        attr=None,
        target=_f32([[1, 0, 0], [0, 1, 0], [0, 0, 1]], dev, (1, 3, 3)),
        init=torch.full((1, 3, 3), 0.5, dtype=torch.float32, device=dev),
        steps=120, learning_rate=0.05, log_every=10)


def _xy_mask(V, dev):
    return torch.tensor([1.0, 1.0, 0.0, 0.0], device=dev).repeat(V).view(1, V, 4)


def pose_scene(dev=None) -> Scene:
    """PoseFitExample/main.swift:22-84: a quad of two triangles, 64x64, solid
    red, target +-0.4 NDC, start shifted and squashed, 300 steps at lr 0.01."""
    dev = dev or _dev()
    return Scene(
        kind="pose", size=64,
        tri=torch.tensor([[0, 1, 2], [0, 2, 3]], dtype=torch.int32, device=dev),
        pos=None,
        attr=_f32([[0.95, 0.2, 0.2]] * 4, dev, (1, 4, 3)),
        target=_f32([[-0.4, 0.4, 0, 1], [0.4, 0.4, 0, 1], [0.4, -0.4, 0, 1],
                     [-0.4, -0.4, 0, 1]], dev, (1, 4, 4)),
        init=_f32([[-0.25, 0.55, 0, 1], [0.55, 0.55, 0, 1], [0.55, -0.25, 0, 1],
                   [-0.25, -0.25, 0, 1]], dev, (1, 4, 4)),
        steps=300, learning_rate=0.01, mask=_xy_mask(4, dev))


def hexagon_pos(center, radius, dev) -> torch.Tensor:
    """MeshFitExample/main.swift:24-33: centre vertex, then six outer vertices
    at 0, 60, ..., 300 degrees (angles and coordinates in fp32)."""
    vals = [center[0], center[1], 0.0, 1.0]
    pi = torch.tensor(math.pi, dtype=torch.float32)
    r = torch.tensor(radius, dtype=torch.float32)
    for k in range(6):
        a = torch.tensor(float(k), dtype=torch.float32) * (pi / 3)
        x = torch.tensor(center[0], dtype=torch.float32) + r * torch.cos(a)
        y = torch.tensor(center[1], dtype=torch.float32) + r * torch.sin(a)
        vals += [float(x), float(y), 0.0, 1.0]
    return torch.tensor(vals, dtype=torch.float32, device=dev).view(1, 7, 4)


def mesh_scene(dev=None) -> Scene:
    """MeshFitExample/main.swift:22-87: the 7-vertex / 6-triangle hexagonal
    pie, 96x96, colour-wheel vertex colours, target radius 0.55 at the
    origin, start radius 0.42 at (0.13, -0.09), 400 steps at lr 0.015."""
    dev = dev or _dev()
    return Scene(
        kind="pose", size=96,
        tri=torch.tensor([[0, 1, 2], [0, 2, 3], [0, 3, 4], [0, 4, 5], [0, 5, 6], [0, 6, 1]],
                         dtype=torch.int32, device=dev),
        pos=None,
        attr=_f32([[1.0, 1.0, 1.0], [1.0, 0.2, 0.2], [1.0, 0.9, 0.2], [0.2, 0.9, 0.3],
                   [0.2, 0.9, 0.9], [0.3, 0.4, 1.0], [1.0, 0.3, 0.9]], dev, (1, 7, 3)),
        target=hexagon_pos((0.0, 0.0), 0.55, dev),
        init=hexagon_pos((0.13, -0.09), 0.42, dev),
        steps=400, learning_rate=0.015, mask=_xy_mask(7, dev))


def make_render(sc: Scene):
    """The sample's `render(param)`: rasterize -> interpolate for "color"
    (rast computed once, pos is fixed), plus antialias for "pose"."""
    S = sc.size
    if sc.kind == "color":
        rast, _ = DiffRast.rasterize(sc.pos, sc.tri, resolution=(S, S), gradDB=False)

        def render(attr):
            out, _ = DiffRast.interpolate(attr, rast, sc.tri)
            return out
        return render
    topology = DiffRast.antialiasConstructTopologyHash(sc.tri)

    def render(pos):
        rast, _ = DiffRast.rasterize(pos, sc.tri, resolution=(S, S), gradDB=False)
        interp, _ = DiffRast.interpolate(sc.attr, rast, sc.tri)
        return DiffRast.antialias(interp, rast, pos, sc.tri, topologyHash=topology)
    return render


def run(sc: Scene, steps: Optional[int] = None, log=None, graph: bool = True) -> FitResult:
    """The sample's optimisation: Adam on the parameter for `steps` steps,
    as replays of one captured step (graph=True) or as eager steps."""
    render = make_render(sc)
    target_image = render(sc.target).detach()
    opt = Adam(sc.init.shape, learningRate=sc.learning_rate)
    loop = _optimise_graph if graph else _optimise
    param, losses = loop(sc.init.clone(), render, target_image, opt,
                         sc.steps if steps is None else steps, mask=sc.mask,
                         log_every=sc.log_every, log=log)
    return FitResult(losses, param, sc.target, sc.size)


def color_fit(steps: Optional[int] = None, log=None, graph: bool = True) -> FitResult:
    """Tier 1 (ColorFitExample/main.swift)."""
    return run(color_scene(), steps, log, graph)


def pose_fit(steps: Optional[int] = None, log=None, graph: bool = True) -> FitResult:
    """Tier 2 (PoseFitExample/main.swift)."""
    return run(pose_scene(), steps, log, graph)


def mesh_fit(steps: Optional[int] = None, log=None, graph: bool = True) -> FitResult:
    """Tier 3 (MeshFitExample/main.swift)."""
    return run(mesh_scene(), steps, log, graph)


SAMPLES = {"color": color_fit, "pose": pose_fit, "mesh": mesh_fit}


def main(argv=None) -> int:
    import argparse
    ap = argparse.ArgumentParser(description="inverse-rendering samples on the HIP path")
    ap.add_argument("sample", choices=sorted(SAMPLES))
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--eager", action="store_true",
                    help="run every step's ops eagerly instead of replaying a captured step")
    args = ap.parse_args(argv)
    fn = SAMPLES[args.sample]
    kw = {} if args.steps is None else {"steps": args.steps}
    res = fn(log=print, graph=not args.eager, **kw)
    print(f"first loss {res.losses[0]:.6f}  final loss {res.losses[-1]:.6f}")
    if args.sample != "color":
        d = (res.param - res.target)[0, :, :2].cpu()
        for v in range(d.shape[0]):
            print(f"  v{v}  delta = ({float(d[v, 0]):+.4f}, {float(d[v, 1]):+.4f})")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
