# Type stub for the compiled extension (csrc/bindings.cpp), as the reference's fa/_C.pyi.
import torch

def forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    variant: str = "opt",
) -> torch.Tensor: ...
def forward_lse(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    variant: str = "opt",
) -> tuple[torch.Tensor, torch.Tensor]: ...
def forward_splitkv(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    softmax_scale: float | None = None,
    num_splits: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]: ...
def version() -> str: ...
