"""One training iteration of the FastGS path, in the order of
Orchestrator::train_step (tinygs/src/orchestrator.cu:335-439):

  zero parameter gradients (:351-353) and loss / gradient images (:354-355)
  -> FastGSRasterizer::forward (:371)
  -> losses: L1 weight * grad_scaler, fused SSIM weight * grad_scaler (:763-782);
     with both on, one fused evaluation that assigns the loss / gradient images
     (the zeroing of :354-355 folded in)
  -> FastGSRasterizer::backward with grad_output = loss gradient (:377-380)
  -> SimpleAdam::step(1 / (grad_scaler * accumulate_grad_steps)) (:393-404)

The parameter-gradient zeroing of :351-353 is folded into the backward:
assign mode writes every row; sparse mode (the default here) writes only
rows that received a gradient and hands Adam the row mask, so zero rows are
neither written nor read.

Everything runs on one HIP stream; the only host synchronisation is the one
inside the forward that sizes the instance buffers. With no_sync=True the
first forward reserves an instance capacity (1.25 x its count) and the later
ones do not wait at all (TGS_FORWARD_NO_SYNC), and Adam keeps its step count
on the device (TGS_ADAM_DEVICE_STEP): from the second step on, a step is the
same launch sequence every time and can be captured into a HIP graph
(capture_step) and replayed; check_status() reports a forward that outgrew
the capacity and reserves room for the next forward. step() checks it every
check_interval eager steps (a wait for the device then), so a scene that grew
(more instances after densification or new parameters) fails loudly instead
of training on partial images.
"""
from __future__ import annotations

from .core import DataType, GPUBatchInput, GPUGaussian3d, Image, LossContext, RasterizeContext
from .loss import create_loss, evaluate_l1_ssim
from .optim import create_optimizer
from .rasterizer import create_rasterizer


class TrainStep:
    def __init__(self, scene, l1_weight: float = 0.8, ssim_weight: float = 0.2, grad_scaler: float = 1.0,
                 eps: float = 1e-15, shs_lr: float | None = None, means_lr: float | None = None,
                 max_grad_1: float | None = None, device: str = "cuda", stream=None, sparse_grads: bool = True,
                 no_sync: bool = False, image_dtype: str = DataType.Float32, overlap_adam: bool = False,
                 check_interval: int = 64):
        """image_dtype: float32, or float16 for the fp16-image rasterizer
        (fastgs.cu:143-188) with the fp16 losses; the target is rounded to half.
        overlap_adam (needs sparse_grads): Adam updates the rows without
        gradient on a second stream while the loss and the backward run, then
        the others; the parameters equal those of the sequential step. Off by
        default: on one MI355X at 1M Gaussians the concurrent kernels slow each
        other down more than the overlap hides (1.16 against 0.98 ms per step)."""
        import torch
        self.scene = scene
        self.no_sync = bool(no_sync)
        self._capacity = None   # (instances, tiles) reserved for the no-sync forwards
        self._reserved = False
        self.check_interval = int(check_interval)   # no_sync: eager steps between capacity checks (0: never)
        self._eager_steps = 0
        # sparse_grads: the backward writes only gradient rows that received a
        # gradient and Adam reads only those (the others are zero); same
        # parameters as assigning every row, without moving the zero rows
        self.sparse_grads = bool(sparse_grads)
        self.overlap_adam = bool(overlap_adam)
        if self.overlap_adam and not self.sparse_grads:
            raise ValueError("overlap_adam needs sparse_grads")
        self._side = None   # the second stream and the fork / join events of overlap_adam
        self._fork = self._join = None
        self.stream = stream
        self.gaussians = GPUGaussian3d.from_scene(scene, device)
        self.grads = self.gaussians.gradient_like()
        self.rasterizer = create_rasterizer("fastgs")
        self.rasterizer.set_gaussians(self.gaussians)
        shape = scene.camera.shape
        self.shape = shape
        self.pred = Image.empty(shape, device, image_dtype)
        tdt = torch.float16 if image_dtype == DataType.Float16 else torch.float32
        self.target = Image(shape, image_dtype, torch.from_numpy(scene.target).to(device).to(tdt))
        self.loss_img = Image.empty(shape, device, image_dtype)
        self.grad_img = Image.empty(shape, device, image_dtype)
        self.losses = []
        if l1_weight:
            self.losses.append((create_loss("l1"), float(l1_weight)))
        if ssim_weight:
            self.losses.append((create_loss("fused_ssim"), float(ssim_weight)))
        self.grad_scaler = float(grad_scaler)
        self.optimizer = create_optimizer("simple_adam", self.gaussians, self.grads)
        params = {"epsilon": eps}
        if shs_lr is not None:
            params["shs_lr"] = shs_lr
        if means_lr is not None:
            params["means_lr"] = means_lr
        if max_grad_1 is not None:
            params["max_grad_1"] = max_grad_1
        self.optimizer.set_params(params)
        self.ctx = RasterizeContext(stream=stream, grad_scaler=self.grad_scaler)
        self.ctx.fwd_input = GPUBatchInput.from_camera(scene.camera)
        self.ctx.fwd_output.image = self.pred
        self.ctx.gaussians_grad = self.grads
        self.ctx.grad_output.image = self.grad_img
        self.loss_ctx = LossContext(self.pred, self.target, self.loss_img, self.grad_img, stream)

    @property
    def fused_losses(self) -> bool:
        """Both L1 and SSIM are on: they run as one fused evaluation in
        assign mode (no separate zeroing of the loss / gradient images)."""
        return len(self.losses) == 2

    def zero(self):
        """Zero the loss and loss-gradient images (unless the fused loss
        evaluation assigns them). The parameter gradients are not zeroed here:
        the backward runs in assign mode, which writes every gradient (zero for
        culled Gaussians), equivalent to zero + accumulate."""
        if self.fused_losses:
            return
        import torch
        s = self.stream
        with torch.cuda.stream(s) if s is not None else _null():
            self.loss_img.data.zero_()
            self.grad_img.data.zero_()

    def forward(self):
        if self.no_sync and self._capacity:
            if not self._reserved:   # before the forward: growing drops the previous forward's state
                self.rasterizer.reserve(*self._capacity, self.stream)
                self._reserved = True
            self.rasterizer.forward(self.ctx, no_sync=True)
            return
        self.rasterizer.forward(self.ctx)
        if self.no_sync:
            _, inst, tiles = self.rasterizer.counts()
            self._capacity = (inst + inst // 4 + 4096, tiles)

    def check_status(self):
        """Waits for the queued steps; raises when a no-sync forward needed
        more instances than reserved (its image and gradients are then partial),
        after reserving room (1.25x the count it needed) for the next forward."""
        from . import _lib
        if self.rasterizer.status(clear_capacity_flag=True, stream=self.stream) == _lib.TGS_ERR_CAPACITY:
            _, inst, tiles = self.rasterizer.counts()
            self._capacity = (inst + inst // 4 + 4096, tiles)
            self._reserved = False   # the next forward reserves the new capacity first
            raise RuntimeError(f"a no-sync forward outgrew its instance capacity ({inst} instances needed); "
                               "the capacity was raised for the next step")

    def losses_and_grad(self):
        if self.fused_losses:
            (l1, w1), (_, w2) = self.losses
            evaluate_l1_ssim(l1, self.loss_ctx, w1 * self.grad_scaler, w2 * self.grad_scaler, assign=True)
            return
        for loss, w in self.losses:
            loss.evaluate(self.loss_ctx, w * self.grad_scaler)

    def backward(self, keep_2d: bool = False):
        if self.sparse_grads:
            self.rasterizer.backward(self.ctx, sparse=True, keep_2d=keep_2d)
        else:
            self.rasterizer.backward(self.ctx, assign=True, keep_2d=keep_2d)

    def optimize(self):
        mask = self.rasterizer.grad_row_mask() if self.sparse_grads else None
        # no_sync: the step count on the device too, so a whole step can be captured
        self.optimizer.step(1.0 / self.grad_scaler, self.stream, row_mask=mask, device_step=self.no_sync)

    def fork_adam_unmarked(self):
        """Right after the forward: Adam's rows that receive no gradient (their
        mask comes from the forward's work items) updated on a second stream
        while the loss and the backward run."""
        import torch
        main = self.stream if self.stream is not None else torch.cuda.current_stream()
        if self._side is None:
            self._side = torch.cuda.Stream(device=main.device)   # default priority
            self._fork, self._join = torch.cuda.Event(), torch.cuda.Event()
        rows = self.rasterizer.backward_rows(main)
        self._fork.record(main)
        self._side.wait_event(self._fork)
        self.optimizer.step(1.0 / self.grad_scaler, self._side, row_mask=rows, device_step=self.no_sync,
                            rows="unmarked")
        self._join.record(self._side)
        return rows

    def join_adam_marked(self, rows):
        """After the backward: Adam's other rows with the same step count. Each
        row is updated once, by the same arithmetic as one masked step."""
        import torch
        main = self.stream if self.stream is not None else torch.cuda.current_stream()
        main.wait_event(self._join)
        self.optimizer.step(1.0 / self.grad_scaler, main, row_mask=rows, device_step=self.no_sync, rows="marked",
                            same_step=True)

    def step(self):
        if self.no_sync and self.check_interval > 0 and self._reserved:
            import torch
            if not torch.cuda.is_current_stream_capturing():
                self._eager_steps += 1
                if self._eager_steps % self.check_interval == 0:
                    self.check_status()
        self.zero()
        self.forward()
        if self.overlap_adam:
            rows = self.fork_adam_unmarked()
            self.losses_and_grad()
            self.backward()
            self.join_adam_marked(rows)
            return
        self.losses_and_grad()
        self.backward()
        self.optimize()

    def capture_step(self):
        """A torch.cuda.CUDAGraph of one step (no_sync mode, after at least two
        eager steps: the first sizes the buffers and reserves the capacity, the
        second seeds the device step count). Replaying it runs a step."""
        import torch
        if not self.no_sync or not self._reserved or self.stream is None:
            raise RuntimeError("capture_step needs no_sync=True, an explicit stream and two eager steps")
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            self.step()
        return g

    # host copies (tests / diagnostics)
    def image(self):
        return self.pred.data.cpu().numpy()

    def grad_image(self):
        return self.grad_img.data.cpu().numpy()

    def params(self):
        g = self.gaussians
        return {"means": g.means().cpu().numpy().reshape(-1), "scales": g.scales().cpu().numpy().reshape(-1),
                "rotations": g.rotations().cpu().numpy().reshape(-1),
                "opacities": g.opacities().cpu().numpy().reshape(-1),
                "sh0": g.sh_coefficient_0().float().cpu().numpy().reshape(-1),
                "sh_rest": g.sh_coefficients_rest().float().cpu().numpy().reshape(-1)}


class _null:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False
