"""Helpers for the GPU parity tests (torch is only the device-memory carrier)."""
import numpy as np
import torch


def dev(a, device="cuda:0"):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def say(msg):
    print(f"[case] {msg}", flush=True)
