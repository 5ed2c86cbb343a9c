"""Run in a fresh process by tests/test_zz_no_alloc.py: the very first
lhq_gemm_w4a16_bf16_noalloc call of the process (where the per-device
scratch address is looked up) is made under torch.cuda.graph capture.  The
graph is replayed three times with new activations, each replay checked bit
for bit against lhq_gemm_w4a16_bf16_ws run eagerly on the same input.
Prints one line per replay and "ok" at the end; exits non-zero on a
mismatch."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def main() -> int:
    import numpy as np
    import torch
    from longhornai_amd import ops
    torch.cuda.set_device(0)
    M, K, N, G = 64, 8192, 8192, 128
    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    q, s, z = ops.w4_buffers(K, N, G, True)
    q.copy_(torch.randint(0, 256, q.shape, dtype=torch.uint8, device="cuda", generator=gen))
    s.copy_((torch.rand(s.shape, device="cuda", generator=gen) * 0.01).half().view(torch.int16))
    z.copy_(torch.randint(-2**31, 2**31 - 1, z.shape, dtype=torch.int32, device="cuda", generator=gen))
    w = ops.W4Weights(q, s, z, K, N, G, True)
    assert ops.lib().lhq_gemm_w4a16_bf16_workspace_bytes(M, N, K, G) > 0
    A = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16)
    C = ops.empty((M, N), np.int16)
    ws = ops.w4a16_bf16_workspace(M, w)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        with torch.cuda.graph(g, stream=st):
            ops.gemm_w4a16_bf16_noalloc(A, w, C)  # the process's first noalloc call
    torch.cuda.current_stream().wait_stream(st)
    torch.cuda.synchronize()
    for rep in range(3):
        A.copy_(torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16).view(torch.int16))
        C.zero_()
        want = ops.host(ops.gemm_w4a16_bf16_ws(A, w, ws), np.uint16)
        g.replay()
        torch.cuda.synchronize()
        same = np.array_equal(ops.host(C, np.uint16), want)
        print(f"replay {rep}: {'bit-identical' if same else 'MISMATCH'}", flush=True)
        if not same:
            return 1
    print("ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
