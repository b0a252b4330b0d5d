"""MI355X-native optimizer step for MiniGPT-style training.

Drop-in replacements for the torch calls of the reference's training loop
(train.py:359-370, 457-491):

    AdamW            for torch.optim.AdamW
    GradScaler       for torch.amp.GradScaler
    clip_grad_norm_  for torch.nn.utils.clip_grad_norm_

plus the loop's host helpers (build_adamw_param_groups, set_optimizer_lr,
cosine_lr, optimizer_completed_steps) and the checkpoint loaders it calls on
resume (load_optimizer_state, load_grad_scaler_state).  The arithmetic runs
in hand-written gfx950 kernels (libmgopt.so, C ABI in include/mgopt.h); there
is no CPU path.

The package directory name contains hyphens, so import it with
importlib.import_module("minigpt-train-infra_amd").
"""

from .adamw import AdamW
from .clip_grad import clip_grad_norm_
from .grad_scaler import GradScaler
from .schedule import build_adamw_param_groups, cosine_lr, optimizer_completed_steps, set_optimizer_lr
from .state_load import load_grad_scaler_state, load_optimizer_state
from . import paramsets

__all__ = [
    "AdamW",
    "GradScaler",
    "clip_grad_norm_",
    "build_adamw_param_groups",
    "cosine_lr",
    "set_optimizer_lr",
    "optimizer_completed_steps",
    "load_optimizer_state",
    "load_grad_scaler_state",
    "paramsets",
]
