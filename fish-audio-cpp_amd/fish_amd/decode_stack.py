"""Decode-step linear stack of the DualAR slow transformer on the W8A8 path.

Mirrors the per-layer call order of DualAREngine::decode_step
(src/engine/dual_ar_engine.cc:576-648) with attention omitted (the o_proj
input is the q slice of the qkv output):

    rms_norm+quant -> qkv -> quant -> o -> residual+rms_norm+quant
    -> gate_up -> silu*mul+quant -> down -> (residual+rms_norm+quant of the
    next layer; a plain residual after the last)

Each residual add is fused into the RMSNorm + quant launch that follows it
(fa_residual_rms_norm_quant), so a layer takes nine launches, two of which
(the o-input copy and its quantizer) stand in for attention.

gate_up is w1 and w3 stacked into one [2 * 9728, 2560] weight (exact when the
two share their input quantization, i.e. no per-weight smooth_inv).
Weights are synthetic (N(0, 0.02) fp16, quantized group-wise on the device).
Every layer owns its own weights, so a 36-layer pass streams ~3.6 GB and
never runs out of the 256 MB last-level cache.
"""
import torch

from . import ops
from .synth import LAYER_SHAPES

HIDDEN = 2560
FFN = 9728
Q_DIM = 32 * 128


class Linear:
    def __init__(self, K, N, g, gen):
        w = torch.randn((N, K), generator=gen, device="cuda", dtype=torch.float32).mul_(0.02).half()
        self.W, self.scale = ops.quantize_weights_groupwise(w, g)
        self.K, self.N, self.g = K, N, g
        del w

    @property
    def algo_bytes(self):
        # int8 W + fp16 scales (+ fp16 x in and y out per token, added by callers)
        return self.W.numel() + 2 * self.scale.numel()


class DecodeStack:
    def __init__(self, n_layers=36, g=256, tokens=1, seed=0):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        self.g, self.n, self.T = g, n_layers, tokens
        self.layers = []
        for _ in range(n_layers):
            lay = {name: Linear(K, N, g, gen) for name, (K, N) in LAYER_SHAPES.items()}
            lay["attn_norm"] = (1 + 0.1 * torch.randn(HIDDEN, generator=gen, device="cuda")).half()
            lay["ffn_norm"] = (1 + 0.1 * torch.randn(HIDDEN, generator=gen, device="cuda")).half()
            self.layers.append(lay)
        T = tokens
        dev = "cuda"
        self.h = torch.randn((T, HIDDEN), generator=gen, device=dev).half()
        self.h0 = self.h.clone()
        # activations / scratch, allocated once
        self.x_in = {name: torch.randn((T, K), generator=gen, device=dev).half()
                     for name, (K, _) in LAYER_SHAPES.items()}
        self.y = {name: torch.empty((T, N), device=dev, dtype=torch.float16)
                  for name, (_, N) in LAYER_SHAPES.items()}
        self.xq = torch.empty((T, FFN), device=dev, dtype=torch.int8)
        self.xs = torch.empty((T, FFN // 64 + 1), device=dev, dtype=torch.float32)
        self.o_in = torch.empty((T, Q_DIM), device=dev, dtype=torch.float16)
        self.gate = torch.empty((T, FFN), device=dev, dtype=torch.float16)
        self.up = torch.empty((T, FFN), device=dev, dtype=torch.float16)
        lib = ops.lib()
        ops.check(lib.fa_workspace_reserve(max(T, 16), 19456, FFN, g, ops._stream()))

    # -- one W8A8 linear through the drop-in entry point (quant + GEMV/GEMM) --
    def linear(self, lay, name, x, out):
        L = lay[name]
        ops.w8a8_gemm(L.W, L.scale, x, L.g, out=out)

    def run_linears(self, layer_ids=None):
        """configs[1]-style work: the four projections of each layer through
        int8_dequant_gemm_fp16 semantics (dynamic per-(token, group) quant)."""
        for l in (range(self.n) if layer_ids is None else layer_ids):
            lay = self.layers[l]
            for name in LAYER_SHAPES:
                self.linear(lay, name, self.x_in[name], self.y[name])

    def linears_bytes(self):
        tot = 0
        for lay in self.layers:
            for name, (K, N) in LAYER_SHAPES.items():
                tot += lay[name].algo_bytes + 2 * self.T * (K + N)
        return tot

    # -- the full decode-step linear stack with fused prologues --
    def run_stack(self):
        g, T = self.g, self.T
        l_ = ops.lib()
        s = ops._stream()
        G2560 = (HIDDEN + g - 1) // g
        for li, lay in enumerate(self.layers):
            # (previous layer's down residual +) attention_norm + quant -> wqkv
            if li == 0:
                ops.check(l_.fa_rms_norm_quant(self.h.data_ptr(), lay["attn_norm"].data_ptr(),
                                               1e-6, None, None, g, self.xq.data_ptr(),
                                               self.xs.data_ptr(), None, T, HIDDEN, s))
            else:
                ops.check(l_.fa_residual_rms_norm_quant(
                    self.h.data_ptr(), self.y["down"].data_ptr(), lay["attn_norm"].data_ptr(),
                    1e-6, None, None, g, self.xq.data_ptr(), self.xs.data_ptr(), None, T, HIDDEN,
                    s))
            L = lay["qkv"]
            ops.check(l_.fa_w8a8_gemm_quantized(L.W.data_ptr(), L.scale.data_ptr(), g,
                                                self.xq.data_ptr(), self.xs.data_ptr(),
                                                self.y["qkv"].data_ptr(), L.N, T, L.K, s))
            # attention omitted: o input is the q slice of the qkv output
            self.o_in.copy_(self.y["qkv"][:, :Q_DIM])
            ops.check(l_.fa_quantize_activations(self.o_in.data_ptr(), None, None,
                                                 self.xq.data_ptr(), self.xs.data_ptr(), T, Q_DIM,
                                                 g, s))
            L = lay["o"]
            ops.check(l_.fa_w8a8_gemm_quantized(L.W.data_ptr(), L.scale.data_ptr(), g,
                                                self.xq.data_ptr(), self.xs.data_ptr(),
                                                self.y["o"].data_ptr(), L.N, T, L.K, s))
            # o residual + ffn_norm + quant -> w1|w3
            ops.check(l_.fa_residual_rms_norm_quant(
                self.h.data_ptr(), self.y["o"].data_ptr(), lay["ffn_norm"].data_ptr(), 1e-6, None,
                None, g, self.xq.data_ptr(), self.xs.data_ptr(), None, T, HIDDEN, s))
            L = lay["gate_up"]
            ops.check(l_.fa_w8a8_gemm_quantized(L.W.data_ptr(), L.scale.data_ptr(), g,
                                                self.xq.data_ptr(), self.xs.data_ptr(),
                                                self.y["gate_up"].data_ptr(), L.N, T, L.K, s))
            if T == 1:
                gate_p = self.y["gate_up"].data_ptr()
                up_p = gate_p + 2 * FFN
            else:
                self.gate.copy_(self.y["gate_up"][:, :FFN])
                self.up.copy_(self.y["gate_up"][:, FFN:])
                gate_p, up_p = self.gate.data_ptr(), self.up.data_ptr()
            ops.check(l_.fa_silu_mul_quant(gate_p, up_p, None, None, g, self.xq.data_ptr(),
                                           self.xs.data_ptr(), None, T, FFN, s))
            L = lay["down"]
            ops.check(l_.fa_w8a8_gemm_quantized(L.W.data_ptr(), L.scale.data_ptr(), g,
                                                self.xq.data_ptr(), self.xs.data_ptr(),
                                                self.y["down"].data_ptr(), L.N, T, L.K, s))
        # the last layer's down residual
        ops.check(l_.fa_residual_add(self.h.data_ptr(), self.y["down"].data_ptr(), T * HIDDEN, s))
        del G2560

    def stack_bytes(self):
        """Algorithmic bytes of one stack pass: int8 W + fp16 scales of all
        linears + gamma + fp16 activations in/out of each linear."""
        tot = self.linears_bytes()
        tot += self.n * 2 * (2 * HIDDEN)
        return tot

    def capture(self, fn):
        """HIP graph of fn() (all launches are on torch's current stream)."""
        fn()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            fn()
        torch.cuda.synchronize()
        return g
