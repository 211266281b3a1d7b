"""Element types of the op inputs: every op takes shape["dtype"] = "fp16" (default, the reference's type) or "bf16"."""
import numpy as np
import torch

DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}


def cast16(a, dtype="fp16", device="cpu"):
    """A float32 NumPy array rounded to fp16 or bf16 (to nearest even) as a torch tensor on `device`."""
    if dtype == "fp16":
        return torch.from_numpy(a.astype(np.float16)).to(device)
    if dtype == "bf16":
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(device)
    raise ValueError(f"unknown dtype {dtype!r}")
