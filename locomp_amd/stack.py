"""SmolLM2-135M-shaped decode step on the quantized linears (hidden 576,
intermediate 1536, 30 layers, vocabulary 49152), with random int4 g32
weights: the caller of the hot path that examples/54_smollm2_inference.py
runs per token (:494-574), with its `_matvec` calls (:491-492) replaced by
the library's dequant-matmul.

A step is the list of `links` of one token, launched back to back on one
stream (captured in a HIP graph by the bench):

* unchained (`chain=False`): every linear reads a fixed activation vector
  (q, k, v, o, gate, up, down per layer, or q|k|v and gate|up fused when
  `fused`), then the LM head;
* chained (`chain=True`, implies fused q|k|v and the SiLU * mul epilogue):
  per layer RMSNorm (with the residual add of the previous layer's down
  projection) -> q|k|v -> o (on the q part, standing in for attention) ->
  residual add + RMSNorm -> gate|up with SiLU * mul -> down; after the
  layers a residual add + final RMSNorm and the LM head (tied embeddings,
  examples/54:569-574).  Attention, RoPE and the KV cache are not on the
  quantized path and are left out.

* chained and fused (`fuse_norm=True`, implies `chain`): the same step in
  4 launches per layer instead of 6, through
  `locomp_amd_dequant_matvec_int4_fused`: rmsnorm(H) -> q|k|v, o + H -> H,
  rmsnorm(H) -> gate|up with SiLU * mul, down + H -> H, and after the
  layers rmsnorm(H) -> LM head.

`keep_host=True` keeps host copies of every weight, scale and norm weight,
so that a test can recompute each link from the device's own inputs.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, synth

HIDDEN, INTER, VOCAB, LAYERS = 576, 1536, 49152, 30
RMS_EPS = 1e-5   # examples/54_smollm2_inference.py:31


class Link:
    """One launch of the step.  kind "matvec": O = X @ deq(W)^T (or, with
    `epi`, silu(gate) * up of interleaved gate|up rows); with `gamma` the
    matmul takes rmsnorm(X) * gamma, with `res` O = ... + res (res is O: the
    hidden state updated in place); kind "norm": H += R (if R),
    Y = rmsnorm(H) * gamma."""

    gamma = None
    res = None

    def __init__(self, kind, **kw):
        self.kind = kind
        self.__dict__.update(kw)


class DecodeStack:
    def __init__(self, seed=0, G=32, fused=False, silu=False, chain=False, f32=False,
                 head=True, keep_host=False, fuse_norm=False):
        import torch
        self.torch = torch
        self.lib = _lib.load()
        self.G = G
        if fuse_norm:
            chain = True
        self.chain = chain
        self.fuse_norm = fuse_norm
        if chain:
            fused = silu = True
        self.dt = _lib.F32 if f32 else _lib.F16
        self.np_dt = np.float32 if f32 else np.float16
        tdt = torch.float32 if f32 else torch.float16
        self.es = 4 if f32 else 2
        rng = np.random.default_rng(seed)
        self.links: list[Link] = []
        self.algo_bytes = 0
        self.host = {} if keep_host else None

        def dev(a):
            return torch.from_numpy(np.ascontiguousarray(a)).cuda()

        def buf(n):
            return torch.zeros(n, dtype=tdt, device="cuda")

        def linear(name, N, K, x, out_n=None, epi=False, norm_w=False, res=None):
            W = synth.int4_weights(rng, N, K)
            S = synth.scales(rng, N, K // G, 0.001, 0.01)
            O = res if res is not None else buf(out_n if out_n is not None else (N // 2 if epi else N))
            g = rng.uniform(0.5, 1.5, K).astype(self.np_dt) if norm_w else None
            self.links.append(Link("matvec", name=name, N=N, K=K, W=dev(W), S=dev(S), O=O, X=x, epi=epi,
                                   gamma=dev(g) if norm_w else None, res=res))
            if keep_host:
                self.host[len(self.links) - 1] = (W, S) if g is None else (W, S, g)
            self.algo_bytes += W.nbytes + S.nbytes + (K + O.numel()) * self.es
            if norm_w:
                self.algo_bytes += K * self.es
            if res is not None:
                self.algo_bytes += O.numel() * self.es
            return O

        def norm(name, H, R, Y):
            g = rng.uniform(0.5, 1.5, HIDDEN).astype(self.np_dt)
            self.links.append(Link("norm", name=name, H=H, R=R, gamma=dev(g), Y=Y))
            if keep_host:
                self.host[len(self.links) - 1] = g
            # H (+ R, + H written back) + gamma + Y
            self.algo_bytes += HIDDEN * self.es * (4 if R is not None else 3)

        if not chain:
            xs = {K: dev(synth.activations(rng, 1, K, dtype=self.np_dt)) for K in (HIDDEN, INTER)}
            self.xs = xs
            for layer in range(LAYERS):
                if fused:
                    linear(f"{layer}.qkv", 960, HIDDEN, xs[HIDDEN])
                    linear(f"{layer}.o", HIDDEN, HIDDEN, xs[HIDDEN])
                    linear(f"{layer}.gate_up", 2 * INTER, HIDDEN, xs[HIDDEN], epi=silu)
                    linear(f"{layer}.down", HIDDEN, INTER, xs[INTER])
                else:
                    for name, (N, K) in zip(("q", "k", "v", "o", "gate", "up", "down"),
                                            synth.SMOLLM2_LAYER):
                        linear(f"{layer}.{name}", N, K, xs[K])
            if head:
                linear("lm_head", VOCAB, HIDDEN, xs[HIDDEN])
        elif fuse_norm:
            self.H = dev(synth.activations(rng, 1, HIDDEN, dtype=self.np_dt).reshape(HIDDEN))
            self.H0 = self.H.clone()
            for layer in range(LAYERS):
                qkv = linear(f"{layer}.input_norm+qkv", 960, HIDDEN, self.H, norm_w=True)
                linear(f"{layer}.o+residual", HIDDEN, HIDDEN, qkv, res=self.H)
                h = linear(f"{layer}.post_attention_norm+gate_up", 2 * INTER, HIDDEN, self.H,
                           epi=True, norm_w=True)
                linear(f"{layer}.down+residual", HIDDEN, INTER, h, res=self.H)
            if head:
                linear("final_norm+lm_head", VOCAB, HIDDEN, self.H, norm_w=True)
        else:
            # the hidden state starts as a random vector (the embedding row)
            self.H = dev(synth.activations(rng, 1, HIDDEN, dtype=self.np_dt).reshape(HIDDEN))
            self.H0 = self.H.clone()
            NB = buf(HIDDEN)
            R = None
            for layer in range(LAYERS):
                norm(f"{layer}.input_norm", self.H, R, NB)
                qkv = linear(f"{layer}.qkv", 960, HIDDEN, NB)
                o = linear(f"{layer}.o", HIDDEN, HIDDEN, qkv)          # reads the q part
                norm(f"{layer}.post_attention_norm", self.H, o, NB)
                h = linear(f"{layer}.gate_up", 2 * INTER, HIDDEN, NB, epi=True)
                R = linear(f"{layer}.down", HIDDEN, INTER, h)
            norm("final_norm", self.H, R, NB)
            if head:
                linear("lm_head", VOCAB, HIDDEN, NB)
        self.R = 1
        torch.cuda.synchronize()

    def reset(self):
        """Restore the chained hidden state (the links update it in place)."""
        if self.chain:
            self.H.copy_(self.H0)

    def run_link(self, j, stream):
        vp = ctypes.c_void_p
        L = self.links[j]
        if L.kind == "norm":
            rc = self.lib.locomp_amd_rms_norm(vp(L.H.data_ptr()), vp(L.R.data_ptr()) if L.R is not None else None,
                                              vp(L.gamma.data_ptr()), vp(L.Y.data_ptr()), 1, HIDDEN,
                                              RMS_EPS, self.dt, stream)
        elif L.gamma is not None or L.res is not None:
            rc = self.lib.locomp_amd_dequant_matvec_int4_fused(
                vp(L.X.data_ptr()), vp(L.W.data_ptr()), vp(L.S.data_ptr()), vp(L.O.data_ptr()),
                L.K, L.K // 2, L.K // self.G, self.G, L.N, 1, self.dt, _lib.F16, self.dt,
                vp(L.gamma.data_ptr()) if L.gamma is not None else None, RMS_EPS,
                vp(L.res.data_ptr()) if L.res is not None else None, 1 if L.epi else 0, stream)
        elif L.epi:
            rc = self.lib.locomp_amd_dequant_matvec_int4_silu_mul(
                vp(L.X.data_ptr()), vp(L.W.data_ptr()), vp(L.S.data_ptr()), vp(L.O.data_ptr()),
                L.K, L.K // 2, L.K // self.G, self.G, L.N // 2, 1, self.dt, _lib.F16, self.dt, stream)
        else:
            rc = self.lib.locomp_amd_dequant_matvec_int4(
                vp(L.X.data_ptr()), vp(L.W.data_ptr()), vp(L.S.data_ptr()), vp(L.O.data_ptr()),
                L.K, L.K // 2, L.K // self.G, self.G, L.N, 1, self.dt, _lib.F16, self.dt, stream)
        if rc != 0:
            raise RuntimeError(f"{L.name}: launch failed: {rc}")

    def launch(self, i, stream):
        for j in range(len(self.links)):
            self.run_link(j, stream)

    @property
    def gemvs(self):
        return sum(1 for L in self.links if L.kind == "matvec")
