#!/usr/bin/env python3
"""Device-to-device copy rates of one MI355X at the sizes of the Q8_0 workload (64 MiB in) and of a large tensor:
the achievable HBM rate a streaming kernel of that size is compared with. Inputs rotate over enough copies to pass
the 256 MB Infinity Cache, so every launch reads HBM; HIP events around 50 (20) back-to-back launches."""
import torch


def rate(fn, reps):
    fn(0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(reps):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def main():
    n = 4096 * 4096
    src = [torch.randn(n, device="cuda") for _ in range(8)]
    dst = [torch.empty(n, device="cuda") for _ in range(8)]
    ms = rate(lambda i: dst[i % 8].copy_(src[i % 8]), 50)
    print("copy 64 MiB -> 64 MiB   %.4f ms  %.2f TB/s" % (ms, 2 * n * 4 / ms / 1e9))
    big = [torch.randn(8 * n, device="cuda") for _ in range(2)]
    bdst = [torch.empty(8 * n, device="cuda") for _ in range(2)]
    ms = rate(lambda i: bdst[i % 2].copy_(big[i % 2]), 20)
    print("copy 512 MiB -> 512 MiB %.4f ms  %.2f TB/s" % (ms, 2 * 8 * n * 4 / ms / 1e9))


if __name__ == "__main__":
    main()
