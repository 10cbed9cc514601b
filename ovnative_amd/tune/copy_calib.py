"""Plain device copy of known size for FETCH_SIZE / WRITE_SIZE calibration."""
import torch
torch.cuda.set_device(0)
n = 64 * 1024 * 1024 // 4
a = torch.randn(n, device='cuda'); b = torch.empty_like(a)
for _ in range(10):
    b.copy_(a)
torch.cuda.synchronize()
print("copied 64 MiB x10")
