"""The config-5 network -- linear + gelu layers, mse loss, Nesterov SGD --
composed over the C ABI the way the reference's nn module composes it.

Each linear layer is matmul then a broadcast bias add (the reference's
pg_ag_linear_forward, nn.c:117-125, with W stored [in, out]); gelu sits
between layers; the loss is pg_ag_mse(out, target, mean=True).  A step is
forward, pg_backward, pg_sgd_step over every W and b (registered W_l, b_l
in layer order), and leaves the grads to the next pg_sgd_zero_grad.

dtype F32 runs the reference's own f32 graph (pg_ag_matmul).  BF16/F16 run
the layer's matmul through pg_amd_ag_matmul16: f32 master weights and
activations, GEMM operands rounded to the 16-bit dtype, f32 accumulation;
the 16-bit weight copy is rewritten by pg_sgd_step in the update pass.
With fused=True (16-bit only) each layer is one pg_amd_ag_linear16 node --
the same arithmetic with bias and gelu in the GEMM epilogue and the bias
grad, gelu' and the 16-bit grad cast in one backward pass.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .capi import F32, PgLib, SgdCfg, shape_arg

ACT_NONE, ACT_RELU, ACT_GELU = 0, 1, 2  # PG_ACT_* (backend/cpu/gemm.h:37-39)


class Mlp:
    def __init__(self, lib: PgLib, Ws, bs, dtype: int = F32,
                 sgd=(0.01, 0.9, 0.0, 1e-4, True), fused: bool = False):
        """Ws, bs: lists of parameter nodes (f32 leaves with requires_grad),
        W_l [d_l, d_{l+1}], b_l [d_{l+1}]; the optimiser retains them."""
        if fused and dtype == F32:
            raise ValueError("fused layers run 16-bit GEMM operands (dtype F16 or BF16)")
        self.lib, self.dtype, self.fused = lib, dtype, fused
        self.Ws, self.bs = list(Ws), list(bs)
        self.opt = lib.pg_sgd_new(C.byref(SgdCfg(*sgd)))
        if not self.opt:
            raise RuntimeError("pg_sgd_new failed")
        for w, b in zip(self.Ws, self.bs):
            if lib.pg_sgd_add_param(self.opt, w) != 0 or lib.pg_sgd_add_param(self.opt, b) != 0:
                raise RuntimeError("pg_sgd_add_param failed")

    @classmethod
    def from_arrays(cls, lib: PgLib, Ws, bs, dtype: int = F32, **kw) -> "Mlp":
        return cls(lib, [lib.var(w) for w in Ws], [lib.var(b) for b in bs], dtype, **kw)

    @classmethod
    def seeded(cls, lib: PgLib, dims, dtype: int = F32, **kw) -> "Mlp":
        """W_l ~ U[-1/sqrt(d_l), 1/sqrt(d_l)] from the library RNG in layer
        order, biases zero (nn.c:104)."""
        Ws, bs = [], []
        for i in range(len(dims) - 1):
            lim = 1.0 / float(np.sqrt(dims[i]))
            nd, sh = shape_arg((dims[i], dims[i + 1]))
            Ws.append(lib._check(lib.pg_var_uniform(nd, sh, -lim, lim, True)))
            nd, sh = shape_arg((dims[i + 1],))
            bs.append(lib._check(lib.pg_var_zeros(nd, sh, True)))
        return cls(lib, Ws, bs, dtype, **kw)

    def _matmul(self, h: int, w: int) -> int:
        if self.dtype == F32:
            return self.lib.op("matmul", h, w)
        return self.lib._check(self.lib.pg_amd_ag_matmul16(h, w, self.dtype))

    def forward(self, x: int):
        """Output node and the intermediate nodes to free after the step."""
        L = self.lib
        h, made = x, []
        if self.fused:
            for i, (w, b) in enumerate(zip(self.Ws, self.bs)):
                act = ACT_GELU if i + 1 < len(self.Ws) else ACT_NONE
                h = L._check(L.pg_amd_ag_linear16(h, w, b, act, self.dtype))
                made.append(h)
            return h, made
        for i, (w, b) in enumerate(zip(self.Ws, self.bs)):
            mm = self._matmul(h, w)
            made.append(mm)
            z = L.op("add", mm, b)
            made.append(z)
            if i + 1 < len(self.Ws):
                h = L.op("gelu", z)
                made.append(h)
            else:
                h = z
        return h, made

    def step(self, x: int, target: int, keep_loss: bool = False):
        """One training step.  Returns the loss node if keep_loss (the caller
        frees it), else None.  Grads stay readable until the next step."""
        L = self.lib
        L.pg_sgd_zero_grad(self.opt)
        out, made = self.forward(x)
        loss = L._check(L.pg_ag_mse(out, target, True))
        L.pg_backward(loss)
        L.pg_sgd_step(self.opt)
        for n in reversed(made):
            L.pg_node_free(n)
        if keep_loss:
            return loss
        L.pg_node_free(loss)
        return None

    def free(self) -> None:
        if self.opt:
            self.lib.pg_sgd_free(self.opt)
            self.opt = None
        for n in self.Ws + self.bs:
            self.lib.pg_node_free(n)
        self.Ws, self.bs = [], []
