"""AdamW on the libnoise_amd kernel (torch.optim.AdamW semantics, as train/val/eggroll.py:205 builds it).

When the parameters are views that exactly tile one flat fp32 buffer (a `noise_amd.model.GPT`
and its gradients from `Eggroll`), the whole update is one launch; otherwise one launch per
parameter. `lr` may be changed between steps through `param_groups` like any torch optimizer
(the reference's warmdown writes `group['lr']`, eggroll.py:208-212).
"""
import torch

from . import kernels as K


def _flat_base(tensors):
    """The flat buffer the tensors tile exactly, in order, or None."""
    if not tensors:
        return None
    base = tensors[0]
    storage = base.untyped_storage().data_ptr()
    off = base.storage_offset()
    for t in tensors:
        if (t.untyped_storage().data_ptr() != storage or t.storage_offset() != off or not t.is_contiguous()):
            return None
        off += t.numel()
    total = off - tensors[0].storage_offset()
    return torch.empty(0, dtype=base.dtype, device=base.device).set_(
        base.untyped_storage(), tensors[0].storage_offset(), (total,))


class AdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.0):
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))
        self._flat = {}  # group index -> moments of a flat group

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for gi, group in enumerate(self.param_groups):
            params = [p for p in group['params'] if p.grad is not None]
            if not params:
                continue
            beta1, beta2 = group['betas']
            state = self._flat.setdefault(gi, {})
            pflat = _flat_base(params)
            gflat = _flat_base([p.grad for p in params])
            if pflat is not None and gflat is not None:
                if 'exp_avg' not in state or state['exp_avg'].numel() != pflat.numel():
                    state['exp_avg'] = torch.zeros_like(pflat)
                    state['exp_avg_sq'] = torch.zeros_like(pflat)
                    state['step'] = 0
                state['step'] += 1
                K.adamw(pflat, gflat, state['exp_avg'], state['exp_avg_sq'], group['lr'], beta1, beta2,
                        group['eps'], group['weight_decay'], state['step'])
                continue
            for p in params:
                st = self.state[p]
                if not st:
                    st['exp_avg'] = torch.zeros_like(p)
                    st['exp_avg_sq'] = torch.zeros_like(p)
                    st['step'] = 0
                st['step'] += 1
                K.adamw(p, p.grad.contiguous(), st['exp_avg'], st['exp_avg_sq'], group['lr'], beta1, beta2,
                        group['eps'], group['weight_decay'], st['step'])
        return loss
