"""Decode-step linear stack of the DualAR slow transformer on the W8A8 path.

Mirrors the per-layer call order of DualAREngine::decode_step
(src/engine/dual_ar_engine.cc:576-648) with attention omitted (the o_proj
input is the q slice of the qkv output):

    residual + rms_norm + quant -> qkv -> quant -> o -> residual + rms_norm
    + quant -> gate_up -> silu*mul + quant -> down -> (the next layer's
    residual; a plain residual add after the last)

Every prologue and the SwiGLU product are fused into the linears
(fa_w8a8_gemm_rms, fa_w8a8_gemm, fa_w8a8_gemm_swiglu), so a layer takes four
launches at one token.

gate_up is w1 and w3 with rows interleaved (row 2i = w1 row i, row 2i+1 = w3
row i) into one [2 * 9728, 2560] weight, so one GEMV wave holds both halves of
an FFN column and its epilogue forms silu(gate) * up directly; exact when the
two share their input quantization, i.e. no per-weight smooth_inv.

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


def smooth_factors(K, gen):
    """AWQ-style per-channel smooth_inv (log-normal around 1, fp16), as the
    reference exporter attaches to every calibrated wqkv / w1 / w3
    (tools/step2_export_w8a8.py:477)."""
    z = torch.randn(K, generator=gen, device="cuda").mul_(0.5).clamp_(-1.6, 1.6)
    return torch.exp(z).half()


class DecodeStack:
    """awq=False: synthetic un-calibrated weights; gate_up is the
    row-interleaved w1 / w3 pair.  awq=True: the calibrated layout a real
    dual_ar.bin carries -- wqkv, w1 and w3 each with their own smooth_inv
    (so w1 and w3 see different int8 inputs and stay separate weights)."""

    def __init__(self, n_layers=36, g=256, tokens=1, seed=0, awq=False):
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed)
        self.g, self.n, self.T, self.awq = g, n_layers, tokens, awq
        self.layers = []
        for _ in range(n_layers):
            if awq:
                lay = {"qkv": Linear(HIDDEN, 6144, g, gen), "o": Linear(Q_DIM, HIDDEN, g, gen),
                       "w1": Linear(HIDDEN, FFN, g, gen), "w3": Linear(HIDDEN, FFN, g, gen),
                       "down": Linear(FFN, HIDDEN, g, gen)}
                for name in ("qkv", "w1", "w3"):
                    lay[name + "_smooth"] = smooth_factors(HIDDEN, gen)
            else:
                lay = {name: Linear(K, N, g, gen) for name, (K, N) in LAYER_SHAPES.items()}
            lay["attn_norm"] = (1 + 0.1 * torch.randn(HIDDEN, generator=gen, device="cuda")).half()
            lay["ffn_norm"] = (1 + 0.1 * torch.randn(HIDDEN, generator=gen, device="cuda")).half()
            self.layers.append(lay)
        T = tokens
        dev = "cuda"
        self.h = torch.randn((T, HIDDEN), generator=gen, device=dev).half()
        self.h0 = self.h.clone()
        self.h_alt = torch.empty_like(self.h)
        # activations / scratch, allocated once
        self.x_in = {name: torch.randn((T, K), generator=gen, device=dev).half()
                     for name, (K, _) in LAYER_SHAPES.items()}
        self.y = {name: torch.empty((T, N), device=dev, dtype=torch.float16)
                  for name, (_, N) in LAYER_SHAPES.items()}
        self.xq = torch.empty((T, FFN), device=dev, dtype=torch.int8)
        self.xs = torch.empty((T, FFN // 64 + 1), device=dev, dtype=torch.float32)
        self.o_in = torch.empty((T, Q_DIM), device=dev, dtype=torch.float16)
        self.act = torch.empty((T, FFN), device=dev, dtype=torch.float16)
        if awq:
            self.gate = torch.empty((T, FFN), device=dev, dtype=torch.float16)
            self.up = torch.empty((T, FFN), device=dev, dtype=torch.float16)
        lib = ops.lib()
        ops.check(lib.fa_workspace_reserve(max(T, 16), 19456, FFN, g, ops._stream()))

    # -- one W8A8 linear through the drop-in entry point (quant + GEMV/GEMM) --
    def linear(self, lay, name, x, out):
        L = lay[name]
        ops.w8a8_gemm(L.W, L.scale, x, L.g, out=out)

    def run_stack_awq(self):
        """The calibrated (AWQ) layout, four launches per layer:

            qkv      fa_w8a8_gemm_rms         h' = h + down_prev; attention_norm(h') * smooth_qkv
            o        fa_w8a8_gemm             the q slice of qkv's output
            gate_up  fa_w8a8_gemm_swiglu_sep  h'' = h' + o; ffn_norm(h''), quantized once with
                                              smooth_w1 for w1 and once with smooth_w3 for w3;
                                              silu(gate) * up
            down     fa_w8a8_gemm             act

        The same values as run_stack_awq_unfused, which follows the reference's
        separate calls (dual_ar_engine.cc:576-648 with each weight's QuantMeta,
        :253-275)."""
        assert self.awq
        g, T = self.g, self.T
        l_ = ops.lib()
        s = ops._stream()
        cur, nxt = self.h, self.h_alt
        if T == 1:
            o_in = self.y["qkv"]
        for li, lay in enumerate(self.layers):
            L = lay["qkv"]
            resid = None if li == 0 else self.y["down"].data_ptr()
            ops.check(l_.fa_w8a8_gemm_rms(L.W.data_ptr(), L.scale.data_ptr(), g, None,
                                          lay["qkv_smooth"].data_ptr(), cur.data_ptr(), resid,
                                          None if li == 0 else nxt.data_ptr(),
                                          lay["attn_norm"].data_ptr(), 1e-6,
                                          self.y["qkv"].data_ptr(), L.N, T, L.K, s))
            if li != 0:
                cur, nxt = nxt, cur
            if T != 1:
                self.o_in.copy_(self.y["qkv"][:, :Q_DIM])
                o_in = self.o_in
            L = lay["o"]
            ops.check(l_.fa_w8a8_gemm(L.W.data_ptr(), L.scale.data_ptr(), g, None, None,
                                      o_in.data_ptr(), self.y["o"].data_ptr(), L.N, T, L.K, s))
            L1, L3 = lay["w1"], lay["w3"]
            ops.check(l_.fa_w8a8_gemm_swiglu_sep(
                L1.W.data_ptr(), L1.scale.data_ptr(), L3.W.data_ptr(), L3.scale.data_ptr(), g,
                None, lay["w1_smooth"].data_ptr(), None, lay["w3_smooth"].data_ptr(),
                cur.data_ptr(), self.y["o"].data_ptr(), nxt.data_ptr(),
                lay["ffn_norm"].data_ptr(), 1e-6, self.act.data_ptr(), L1.N, T, L1.K, s))
            cur, nxt = nxt, cur
            L = lay["down"]
            ops.check(l_.fa_w8a8_gemm(L.W.data_ptr(), L.scale.data_ptr(), g, None, None,
                                      self.act.data_ptr(), self.y["down"].data_ptr(), L.N, T,
                                      L.K, s))
        ops.check(l_.fa_residual_add(cur.data_ptr(), self.y["down"].data_ptr(), T * HIDDEN, s))
        if cur is not self.h:
            self.h.copy_(cur)

    def run_stack_awq_unfused(self):
        """The calibrated (AWQ) layout, five launches per layer:

            qkv   fa_w8a8_gemm_rms       h' = h + down_prev; attention_norm(h') * smooth_qkv
            o     fa_w8a8_gemm           the q slice of qkv's output
            w1    fa_w8a8_gemm_rms       h'' = h' + o; ffn_norm(h'') * smooth_w1 -> gate
            w3    fa_w8a8_gemm_rms       ffn_norm(h'') * smooth_w3 -> up
            down  fa_w8a8_gemm_silu_mul  silu(gate) * up

        (dual_ar_engine.cc:576-648 with each weight's QuantMeta, :253-275.)"""
        assert self.awq
        g, T = self.g, self.T
        l_ = ops.lib()
        s = ops._stream()
        cur, nxt = self.h, self.h_alt
        if T == 1:
            o_in = self.y["qkv"]
        for li, lay in enumerate(self.layers):
            L = lay["qkv"]
            resid = None if li == 0 else self.y["down"].data_ptr()
            ops.check(l_.fa_w8a8_gemm_rms(L.W.data_ptr(), L.scale.data_ptr(), g, None,
                                          lay["qkv_smooth"].data_ptr(), cur.data_ptr(), resid,
                                          None if li == 0 else nxt.data_ptr(),
                                          lay["attn_norm"].data_ptr(), 1e-6,
                                          self.y["qkv"].data_ptr(), L.N, T, L.K, s))
            if li != 0:
                cur, nxt = nxt, cur
            if T != 1:
                self.o_in.copy_(self.y["qkv"][:, :Q_DIM])
                o_in = self.o_in
            L = lay["o"]
            ops.check(l_.fa_w8a8_gemm(L.W.data_ptr(), L.scale.data_ptr(), g, None, None,
                                      o_in.data_ptr(), self.y["o"].data_ptr(), L.N, T, L.K, s))
            L = lay["w1"]
            ops.check(l_.fa_w8a8_gemm_rms(L.W.data_ptr(), L.scale.data_ptr(), g, None,
                                          lay["w1_smooth"].data_ptr(), cur.data_ptr(),
                                          self.y["o"].data_ptr(), nxt.data_ptr(),
                                          lay["ffn_norm"].data_ptr(), 1e-6, self.gate.data_ptr(),
                                          L.N, T, L.K, s))
            cur, nxt = nxt, cur
            L = lay["w3"]
            ops.check(l_.fa_w8a8_gemm_rms(L.W.data_ptr(), L.scale.data_ptr(), g, None,
                                          lay["w3_smooth"].data_ptr(), cur.data_ptr(), None, None,
                                          lay["ffn_norm"].data_ptr(), 1e-6, self.up.data_ptr(),
                                          L.N, T, L.K, s))
            L = lay["down"]
            ops.check(l_.fa_w8a8_gemm_silu_mul(L.W.data_ptr(), L.scale.data_ptr(), g, None, None,
                                               self.gate.data_ptr(), self.up.data_ptr(),
                                               self.y["down"].data_ptr(), L.N, T, L.K, s))
        ops.check(l_.fa_residual_add(cur.data_ptr(), self.y["down"].data_ptr(), T * HIDDEN, s))
        if cur is not self.h:
            self.h.copy_(cur)

    def awq_stack_bytes(self):
        """Algorithmic bytes of one calibrated-layout pass, counted as the
        reference moves them (both run_stack_awq variants use this count):
        int8 W + fp16 scales, the three smooth_inv vectors, gamma twice, and
        each of the five linears' fp16 activations in and out (silu_mul
        reads gate and up)."""
        tot = 0
        for lay in self.layers:
            for name in ("qkv", "o", "w1", "w3", "down"):
                L = lay[name]
                tot += L.algo_bytes + 2 * self.T * (L.K + L.N)
            tot += 3 * 2 * HIDDEN + 2 * 2 * HIDDEN + 2 * self.T * FFN
        return tot

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
        """Four launches per layer: every linear forms its own int8 input.

            qkv      fa_w8a8_gemm_rms     h' = h + down_prev; attention_norm(h')
            o        fa_w8a8_gemm         the q slice of qkv's output (attention omitted)
            gate_up  fa_w8a8_gemm_swiglu  h'' = h' + o; ffn_norm(h''); silu(gate) * up
            down     fa_w8a8_gemm         act

        The residual stream ping-pongs between two buffers (a fused residual
        write must not overwrite the stream other workgroups still read); the
        result ends in self.h.  Tokens > 1 take the same entry points, which
        then run their prologue and linear as separate launches."""
        g, T = self.g, self.T
        l_ = ops.lib()
        s = ops._stream()
        cur, nxt = self.h, self.h_alt
        if T == 1:
            o_in = self.y["qkv"]            # the q slice is the row's first Q_DIM values
        for li, lay in enumerate(self.layers):
            L = lay["qkv"]
            resid = None if li == 0 else self.y["down"].data_ptr()
            ops.check(l_.fa_w8a8_gemm_rms(L.W.data_ptr(), L.scale.data_ptr(), g, None, None,
                                          cur.data_ptr(), resid,
                                          None if li == 0 else nxt.data_ptr(),
                                          lay["attn_norm"].data_ptr(), 1e-6,
                                          self.y["qkv"].data_ptr(), L.N, T, L.K, s))
            if li != 0:
                cur, nxt = nxt, cur
            if T != 1:
                self.o_in.copy_(self.y["qkv"][:, :Q_DIM])
                o_in = self.o_in
            L = lay["o"]
            ops.check(l_.fa_w8a8_gemm(L.W.data_ptr(), L.scale.data_ptr(), g, None, None,
                                      o_in.data_ptr(), self.y["o"].data_ptr(), L.N, T, L.K, s))
            L = lay["gate_up"]
            ops.check(l_.fa_w8a8_gemm_swiglu(L.W.data_ptr(), L.scale.data_ptr(), g, None, None,
                                             cur.data_ptr(), self.y["o"].data_ptr(),
                                             nxt.data_ptr(), lay["ffn_norm"].data_ptr(), 1e-6,
                                             self.act.data_ptr(), L.N // 2, T, L.K, s))
            cur, nxt = nxt, cur
            L = lay["down"]
            ops.check(l_.fa_w8a8_gemm(L.W.data_ptr(), L.scale.data_ptr(), g, None, None,
                                      self.act.data_ptr(), self.y["down"].data_ptr(), L.N, T,
                                      L.K, s))
        # the last layer's down residual
        ops.check(l_.fa_residual_add(cur.data_ptr(), self.y["down"].data_ptr(), T * HIDDEN, s))
        if cur is not self.h:
            self.h.copy_(cur)

    # -- configs[4] as one device-ordered launch (fa_chain) --
    def build_chain(self):
        """The steps of run_stack (T == 1) as a fa_chain: the same kernels'
        arithmetic and the same buffers, one launch for all 4 * n linears."""
        assert self.T == 1, "the chain serves one-token decode"
        steps = []
        cur, nxt = self.h, self.h_alt
        for li, lay in enumerate(self.layers):
            L = lay["qkv"]
            st = dict(w=L.W, w_scale=L.scale, x=cur, y=self.y["qkv"], gamma=lay["attn_norm"],
                      prologue=2, eps=1e-6)
            if li != 0:
                st.update(x2=self.y["down"], h_out=nxt)
                cur, nxt = nxt, cur
            steps.append(st)
            L = lay["o"]
            steps.append(dict(w=L.W, w_scale=L.scale, x=self.y["qkv"], k=Q_DIM, y=self.y["o"]))
            L = lay["gate_up"]
            steps.append(dict(w=L.W, w_scale=L.scale, x=cur, x2=self.y["o"], h_out=nxt,
                              gamma=lay["ffn_norm"], y=self.act, prologue=2, epilogue=1, eps=1e-6))
            cur, nxt = nxt, cur
            L = lay["down"]
            steps.append(dict(w=L.W, w_scale=L.scale, x=self.act, y=self.y["down"]))
        self._chain_out = cur
        self.chain = ops.Chain(steps, self.g)
        return self.chain

    def run_chain(self, check=True):
        """run_stack's result through one chain launch (+ the last residual add).
        check: wait for the launch and raise if a step's bounded wait gave up
        (the outputs are then incomplete); callers timing back-to-back runs
        pass False and check chain.status() themselves afterwards."""
        if getattr(self, "chain", None) is None:
            self.build_chain()
        self.chain.run()
        if check:
            rc = self.chain.status()
            if rc != 0:
                raise ops.FaError(rc, "decode chain: a step's wait gave up; outputs incomplete")
        cur = self._chain_out
        l_ = ops.lib()
        ops.check(l_.fa_residual_add(cur.data_ptr(), self.y["down"].data_ptr(), HIDDEN,
                                     ops._stream()))
        if cur is not self.h:
            self.h.copy_(cur)

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


CODEBOOK_SIZE = 4096
NUM_CODEBOOKS = 10


class FastDecoder(DecodeStack):
    """The fast (codebook) decoder pass of a frame
    (DualAREngine::fast_codebook_decode_device, dual_ar_engine.cc:772-845):
    4 layers of the slow layer's shapes (dual_ar_config.h:21-31), then the
    final RMSNorm and the int8 output head (codebook_size 4096 x 2560,
    :836-838), run once per codebook -- 10 times per frame.  The layer
    linears are DecodeStack's (four fused launches per layer); the head is
    fa_w8a8_gemm_rms.  Attention, RoPE and the codebook embedding are out of
    scope: each pass starts from the same synthetic hidden state."""

    def __init__(self, g=256, seed=0, n_layers=4):
        super().__init__(n_layers=n_layers, g=g, tokens=1, seed=seed)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(seed + 1000)
        self.head = Linear(HIDDEN, CODEBOOK_SIZE, g, gen)
        self.fast_norm = (1 + 0.1 * torch.randn(HIDDEN, generator=gen, device="cuda")).half()
        self.logits = torch.empty((1, CODEBOOK_SIZE), device="cuda", dtype=torch.float16)

    def run_pass(self):
        """One codebook step: the 4-layer stack from h0, then the head."""
        self.h.copy_(self.h0)
        self.run_stack()
        L = self.head
        ops.check(ops.lib().fa_w8a8_gemm_rms(L.W.data_ptr(), L.scale.data_ptr(), self.g, None,
                                             None, self.h.data_ptr(), None, None,
                                             self.fast_norm.data_ptr(), 1e-6,
                                             self.logits.data_ptr(), L.N, 1, L.K, ops._stream()))

    def run_frame(self):
        for _ in range(NUM_CODEBOOKS):
            self.run_pass()

    def pass_bytes(self):
        """Algorithmic bytes of one pass: the stack's plus the head's W,
        scales, gamma and activations."""
        return self.stack_bytes() + self.head.algo_bytes + 2 * (2 * HIDDEN + CODEBOOK_SIZE)
