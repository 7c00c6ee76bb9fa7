"""Helpers shared by the GPU tests: move oracle arrays to the device."""

import numpy as np
import torch


def to_dev_bf16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(dev)


def state_to_device(st, dev) -> dict:
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return dict(
        k_packed=t(st.k_packed), v_packed=t(st.v_packed),
        k_scale=t(st.k_scale), v_scale=t(st.v_scale),
        k_topk=to_dev_bf16(st.k_topk, dev), v_topk=to_dev_bf16(st.v_topk, dev),
        k_staging=to_dev_bf16(st.k_staging, dev), v_staging=to_dev_bf16(st.v_staging, dev),
        k_window=to_dev_bf16(st.k_window, dev), v_window=to_dev_bf16(st.v_window, dev),
    )
