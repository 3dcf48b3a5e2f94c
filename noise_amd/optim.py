"""AdamW on the libnoise_amd kernel (torch.optim.AdamW semantics, as train/val/eggroll.py:205 builds it).

The per-parameter state has torch.optim.AdamW's own keys and layout -- 'step' (a 0-dim float
tensor), 'exp_avg', 'exp_avg_sq' -- so `state_dict()` / `load_state_dict()` round-trip it like
torch's. When the parameters (and their gradients) are views that exactly tile one flat fp32
buffer (a `noise_amd.model.GPT` and the gradients `Eggroll` sets), every state tensor is a view of
one flat moment buffer laid out the same way and the whole update is one launch; otherwise one
launch per parameter on the same state. `lr` may be changed between steps through `param_groups`
like any torch optimizer (the reference's warmdown writes `group['lr']`, eggroll.py:208-212).
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
        if (t.untyped_storage().data_ptr() != storage or t.storage_offset() != off or not t.is_contiguous()
                or t.dtype != base.dtype or t.device != base.device):
            return None
        off += t.numel()
    total = off - tensors[0].storage_offset()
    return torch.empty(0, dtype=base.dtype, device=base.device).set_(
        base.untyped_storage(), tensors[0].storage_offset(), (total,))


class AdamW(torch.optim.Optimizer):
    def __init__(self, params, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2):
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))

    def _state(self, p):
        st = self.state[p]
        if not st:
            st['step'] = torch.tensor(0.0)
            st['exp_avg'] = torch.zeros_like(p)
            st['exp_avg_sq'] = torch.zeros_like(p)
        return st

    def _flat_moments(self, params, pflat):
        """(exp_avg, exp_avg_sq) flat buffers laid out like pflat whose views are the params'
        state tensors; states that are not such views yet (new, or loaded from a state dict) are
        gathered into fresh buffers first. None if the params are at different steps."""
        states = [self._state(p) for p in params]
        if len({float(st['step']) for st in states}) != 1:
            return None
        flats = []
        for key in ('exp_avg', 'exp_avg_sq'):
            flat = _flat_base([st[key] for st in states])
            if flat is None or flat.numel() != pflat.numel() or flat.device != pflat.device:
                flat = torch.cat([st[key].reshape(-1).to(pflat.device, torch.float32) for st in states])
                off = 0
                for p, st in zip(params, states):
                    st[key] = flat[off:off + p.numel()].view_as(p)
                    off += p.numel()
            flats.append(flat)
        return flats

    @torch.no_grad()
    def step(self, closure=None, unless=None):
        """One update of every parameter with a gradient. unless: a device int32 status; when it
        is not 0 on the device, the launches leave parameters and moments as they are (the host's
        step counts still advance: `rewind()` takes them back)."""
        self._advanced = []
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        for group in self.param_groups:
            params = [p for p in group['params'] if p.grad is not None]
            if not params:
                continue
            beta1, beta2 = group['betas']
            args = (group['lr'], beta1, beta2, group['eps'], group['weight_decay'])
            pflat = _flat_base(params)
            gflat = _flat_base([p.grad for p in params])
            flats = self._flat_moments(params, pflat) if pflat is not None and gflat is not None else None
            if flats is not None:
                for p in params:
                    self.state[p]['step'] += 1
                self._advanced += params
                K.adamw(pflat, gflat, flats[0], flats[1], *args, int(self.state[params[0]]['step']), unless=unless)
                continue
            for p in params:
                st = self._state(p)
                st['step'] += 1
                self._advanced.append(p)
                for key in ('exp_avg', 'exp_avg_sq'):
                    if not st[key].is_contiguous():
                        st[key] = st[key].contiguous()
                K.adamw(p, p.grad.contiguous(), st['exp_avg'], st['exp_avg_sq'], *args, int(st['step']), unless=unless)
        return loss

    def rewind(self):
        """Take back the step counts the last step() advanced (after its `unless` status skipped
        the update on the device)."""
        for p in getattr(self, '_advanced', []):
            self.state[p]['step'] -= 1
        self._advanced = []
