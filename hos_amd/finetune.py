"""Host-side mirror of HOS's full-parameter finetune (FtModel, src/finetune.rs) over the C ABI: every weight
trainable on the device, loss_grad / adamw / step as the LoRA model's (hos_amd.peft.PeftModel)."""
import ctypes

import numpy as np

from ._lib import lib
from .hip_be import Gpu, HosError
from .peft import ModelConfig, _cstruct


class FtModel:
    def __init__(self, gpu: Gpu, cfg: ModelConfig, max_batch=None, max_seq=None):
        self.gpu, self.cfg = gpu, cfg
        c = _cstruct(cfg, max_batch, max_seq)
        h = ctypes.c_void_p()
        rc = lib().hos_ft_create(gpu.h, ctypes.byref(c), ctypes.byref(h))
        if rc:
            raise HosError(rc, "hos_ft_create failed (see stderr)")
        self.h = h
        gpu.adopt(self)

    def close(self):
        if getattr(self, "h", None):
            lib().hos_ft_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _chk(self, rc):
        if rc:
            raise HosError(rc, lib().hos_ft_last_error(self.h).decode())

    def set_tensor(self, name, raw, ggml_type, rows, cols):
        raw = np.ascontiguousarray(raw).view(np.uint8).ravel()
        self._chk(lib().hos_ft_set_tensor(self.h, name.encode(), raw.ctypes.data, raw.size, ggml_type, rows, cols))

    def load(self, tensors):
        for name, (raw, t, rows, cols) in tensors.items():
            self.set_tensor(name, raw, t, rows, cols)

    def get(self, name, shape):
        """(value, gradient) of a parameter by GGUF name, GGUF layout."""
        v = np.empty(shape, np.float32)
        g = np.empty(shape, np.float32)
        self._chk(lib().hos_ft_get(self.h, name.encode(), v.ctypes.data, g.ctypes.data))
        return v, g

    def loss_grad(self, ids, targets):
        ids = np.ascontiguousarray(ids, np.int32)
        tg = np.ascontiguousarray(targets, np.int32)
        B, T = ids.shape
        loss = ctypes.c_float()
        self._chk(lib().hos_ft_loss_grad(self.h, ids.ctypes.data, tg.ctypes.data, B, T, ctypes.byref(loss)))
        return loss.value

    def adamw(self, lr, wd=0.0):
        self._chk(lib().hos_ft_adamw(self.h, lr, wd))

    def step(self, ids, targets, lr, wd=0.0):
        loss = self.loss_grad(ids, targets)
        self.adamw(lr, wd)
        return loss

    def step_dev(self, ids_dev, tgt_dev, B, T, lr, wd=0.0, loss_dev=None):
        self._chk(lib().hos_ft_step_dev(self.h, ids_dev, tgt_dev, B, T, lr, wd, loss_dev))
