"""DiT-style int8 linear stack (the s3dit int8 block's linears at config-4 shapes).

crates/s3dit/src/block.rs:727-790 (`build_block_steps_i8`) runs every linear
of a DiT block as per-token activation quant + `matmul_i8_dyn`. The
activation is quantized once per distinct input and shared by the linears
that read it. The stack here keeps exactly that int8 work at the synthetic
S3-DiT shapes: M = 1152 tokens (1024 patches of a 64x64 latent at 2x2, plus
128 text tokens), hidden 3840, FFN 10240. Per layer:

    sx, xq = quant(x)                 3840 wide
    qkv    = mm8(xq, Wqkv)            3840 -> 11520 (q|k|v stacked)
    o      = mm8(xq, Wo)              3840 -> 3840
    sx, xq = quant(o)
    h      = mm8(xq, W1)              3840 -> 10240
    sx, xq = quant(h)                 10240 wide
    x      = mm8(xq, W2)              10240 -> 3840 (next layer's input)

Activations are bf16 between linears. Norms, RoPE and the attention core are
f32 work outside the int8 path and are not part of the stack. The out
projection reads the block input's quantized activation in place of the
attention context; the shapes and the int8 work are the block's.

Weights: int8 uniform in [-127, 127]. The per-channel scales are
U(0.5, 1.5) / (73.3 sqrt(K)), which keeps activations O(1) through 30 layers
(73.3 is the standard deviation of a uniform int8). All compute goes through
libbrain_hip.so (bh_quantize_rows_bf16, bh_matmul_i8_dyn). torch only
allocates and captures the step in a HIP graph.

With fuse=True (the default) a linear whose output is quantized next -- the
out projection, and the down projection of every layer but the last (its
output is the next layer's input) -- runs as bh_matmul_i8_dyn_quant, which
gives the same bits as the linear and the quantization called one after the
other.
"""
import torch

from . import ops

DIT_M, DIT_D, DIT_FF, DIT_QKV, DIT_LAYERS = 1152, 3840, 10240, 11520, 30

LINEARS = (("qkv", DIT_D, DIT_QKV), ("o", DIT_D, DIT_D), ("w1", DIT_D, DIT_FF), ("w2", DIT_FF, DIT_D))


def linear_ops(m=DIT_M):
    """Integer ops (2*M*N*K) of one layer's four linears."""
    return sum(2 * m * n * k for _, k, n in LINEARS)


class DitInt8Stack:
    def __init__(self, layers=DIT_LAYERS, m=DIT_M, device="cuda", seed=0, fuse=True):
        self.m, self.layers, self.fuse = m, layers, fuse
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.w = []
        for _ in range(layers):
            lw = {}
            for name, k, n in LINEARS:
                wq = torch.randint(-127, 128, (n, k), dtype=torch.int8, device=device, generator=g).view(torch.int32)
                sw = (torch.rand(n, device=device, generator=g) + 0.5) / (73.3 * k ** 0.5)
                lw[name] = (wq, sw)
            self.w.append(lw)
        self.x = torch.randn(m, DIT_D, device=device, generator=g).to(torch.bfloat16)
        self.x0 = self.x.clone()
        self.qkv = torch.empty(m, DIT_QKV, device=device, dtype=torch.bfloat16)
        self.o = torch.empty(m, DIT_D, device=device, dtype=torch.bfloat16)
        self.h = torch.empty(m, DIT_FF, device=device, dtype=torch.bfloat16)
        self.sx = torch.empty(m, device=device, dtype=torch.float32)
        self.xq = torch.empty(m, DIT_FF // 4, device=device, dtype=torch.int32)
        self.graph = None

    def _mm(self, xq, lw, name, out):
        wq, sw = lw[name]
        ops.matmul_i8(xq, wq, self.sx, sw, None, torch.bfloat16, "dyn", out=out)

    def _mm_quant(self, xq, lw, name, out, xq_out):
        """out = linear(xq), then sx, xq_out = quant(out)."""
        if self.fuse:
            wq, sw = lw[name]
            ops.matmul_i8_quant(xq, wq, self.sx, sw, None, out=out, sx_out=self.sx, xq_out=xq_out)
        else:
            self._mm(xq, lw, name, out)
            ops.quantize_rows_bf16(out, self.sx, xq_out)

    def layer(self, i):
        lw, m = self.w[i], self.m
        xq_d = self.xq.view(-1)[: m * DIT_D // 4].view(m, DIT_D // 4)
        if i == 0 or not self.fuse:  # otherwise the previous layer's down projection quantized x
            ops.quantize_rows_bf16(self.x, self.sx, xq_d)
        self._mm(xq_d, lw, "qkv", self.qkv)
        self._mm_quant(xq_d, lw, "o", self.o, xq_d)
        self._mm(xq_d, lw, "w1", self.h)
        ops.quantize_rows_bf16(self.h, self.sx, self.xq)
        if i + 1 < self.layers:
            self._mm_quant(self.xq, lw, "w2", self.x, xq_d)
        else:
            self._mm(self.xq, lw, "w2", self.x)

    def step(self):
        for i in range(self.layers):
            self.layer(i)

    def capture(self):
        """Record one step (all layers) in a HIP graph on a side stream. The
        split-K workspace of that stream is sized first (a linear whose GEMM
        splits K cannot allocate it during capture)."""
        s = torch.cuda.Stream()
        for _, k, n in LINEARS:
            ops.reserve_workspace(self.m, k, n, s)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.step()  # warm (first-touch) outside the capture
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=s):
            self.step()
        torch.cuda.synchronize()

    def replay(self):
        self.graph.replay()
