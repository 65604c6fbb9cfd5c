"""Synthetic multi-layer MoE decode step on the gfx950 GEMV (batch-1 decode).

Two launch plans compute the same bytes (tested bit-identical):
  fused=True (default): two launches per layer --
    ggml_hip_moe_ffn_gate_up_norm   RMSNorm(x) * norm weight -> q8_1 inside the
                                    gate/up GEMV (+ shared expert, SwiGLU) -> h and
                                    its q8_1 copy hq
    ggml_hip_moe_ffn_down_combine   down GEMV over the picks + shared expert from
                                    hq, x' = x + shared + sum_j w_j o_j
  fused=False: the op-by-op plan below (three launches per layer + one per token).

Per layer, for one token (the op sequence of a ggml MoE FFN block):
  1. gate/up MUL_MAT_ID over the routed experts, fused SwiGLU, with the shared
     expert's gate/up in the same launch             -> h[0..n_used)   and h[n_used]
  2. down MUL_MAT_ID (one activation row per slot), shared expert's down in the
     same launch, reading the fp32 GLU rows and quantizing them to q8_1 inside
     the GEMV                                       -> o[0..n_used) and o_sh
  3. combine x' = x + o_sh + sum_j w_j o_j, fused with the next block's
     ffn_norm (RMSNorm times its norm weight) and the q8_1 quantization of the
     normalized row for the next layer's gate/up launch.
Every launch goes through the C ABI (include/ggml_hip_moe_cache.h); one token is
captured once into a hipGraph and replayed, with routing ids and router
weights copied into fixed device buffers before each replay.

Weights are random valid quantized blocks (uniform codes and scale bits, fp16
block scales set to finite values of realistic magnitude) generated on the GPU:
the GEMV's speed does not depend on the values; numerics are covered by the
parity tests against the CPU oracle.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np

from . import (ACT_DOT_Q8_K, ACT_F32, ACT_Q8_1, ACT_Q8_K, ACT_SHARED_F32, BLOCK, GLU_SWIGLU, KQUANTS, Q2_K, Q3_K, Q4_0, Q4_K, Q5_0, Q5_K, Q6_K, Q8_0, check,
               lib, make_fusion, make_tensor, row_bytes)

# byte offsets of the fp16 block-scale fields per type, and the value written there
_SCALE_FIELDS = {
    Q2_K: ((80, 2e-3), (82, 2e-3)),
    Q3_K: ((108, 2e-4),),
    Q4_K: ((0, 4e-5), (2, 4e-5)),
    Q5_K: ((0, 2e-5), (2, 2e-5)),
    Q6_K: ((208, 5e-6),),
    Q4_0: ((0, 2e-3),),
    Q5_0: ((0, 1e-3),),
    Q8_0: ((0, 2e-4),),
}


def random_expert_tensor(torch, wtype, n_experts, rows, k, gen, device="cuda"):
    """uint8 [n_experts, rows, row_bytes] of valid random blocks of `wtype`."""
    rb = row_bytes(wtype, k)
    t = torch.randint(0, 256, (n_experts, rows, rb), dtype=torch.uint8, device=device, generator=gen)
    bb = BLOCK[wtype][1]
    blocks = t.view(n_experts, rows, rb // bb, bb)
    for off, val in _SCALE_FIELDS[wtype]:
        h = np.array([val], dtype=np.float16).view(np.uint8)
        blocks[..., off] = int(h[0])
        blocks[..., off + 1] = int(h[1])
    return t


class Layer:
    pass


class MoeDecodeModel:
    def __init__(self, torch, n_layers=48, n_experts=512, hidden=4096, ffn=768, n_used=8, wtype=Q2_K,
                 sh_type=Q4_K, seed=0, device="cuda", residual=True, fused=True, shared_q8=True, act="q8_1",
                 mix="pure", hand_off="q8_1"):
        self.torch = torch
        self.fused = fused
        # fused plan: the dots run on q8_1 rows (ggml-CUDA's MMVQ activations, the reference's
        # path) or on q8_K rows (ggml-CPU's MUL_MAT_ID activations for K-quant experts)
        assert act in ("q8_1", "q8_K") and (act == "q8_1" or fused)
        self.act = act
        # fused plan: the gate/up launch writes the shared expert's q8_1 row (32-row shared
        # workgroups) or only its fp32 row, which the down launch quantizes (shared
        # workgroups of a routed one's bytes)
        self.shared_q8 = shared_q8
        # fused plan, q8_1 dots: the gate/up launch hands the GLU rows over as q8_1 blocks (32-row
        # workgroups, one q8_1 block each) or as fp32 rows only (workgroups sized by bytes to the CU
        # count), which every down wave quantizes to q8_1 itself; q8_K dots always take fp32 rows
        assert hand_off in ("q8_1", "f32")
        self.hand_off = hand_off
        self.L, self.E, self.H, self.F, self.U = n_layers, n_experts, hidden, ffn, n_used
        self.wtype, self.sh_type = wtype, sh_type
        # "pure": every routed matrix in wtype; "q2_K_s": llama.cpp's Q2_K_S expert mix -- the
        # ffn_down experts of the first n_layer / 8 layers in Q4_K, the rest in wtype
        assert mix in ("pure", "q2_K_s")
        self.mix = mix
        self.down_types = [Q4_K if mix == "q2_K_s" and l < n_layers // 8 else wtype for l in range(n_layers)]
        self.residual = residual
        self.eps = 1e-6
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        self.layers = []
        keep = []
        for l in range(n_layers):
            ly = Layer()
            ly.down_type = self.down_types[l]
            ly.gate = random_expert_tensor(torch, wtype, n_experts, ffn, hidden, gen, device)
            ly.up = random_expert_tensor(torch, wtype, n_experts, ffn, hidden, gen, device)
            ly.down = random_expert_tensor(torch, ly.down_type, n_experts, hidden, ffn, gen, device)
            ly.sh_gate = random_expert_tensor(torch, sh_type, 1, ffn, hidden, gen, device)[0]
            ly.sh_up = random_expert_tensor(torch, sh_type, 1, ffn, hidden, gen, device)[0]
            ly.sh_down = random_expert_tensor(torch, sh_type, 1, hidden, ffn, gen, device)[0]
            ly.t_up = make_tensor(wtype, hidden, ffn, n_experts, ly.up.data_ptr(), keep=keep)
            ly.t_down = make_tensor(ly.down_type, ffn, hidden, n_experts, ly.down.data_ptr(), keep=keep)
            self.layers.append(ly)
        self._keep = keep
        f32, u8, i32 = torch.float32, torch.uint8, torch.int32
        self.x = torch.zeros((1, hidden), dtype=f32, device=device)          # residual stream
        self.x_next = torch.zeros((1, hidden), dtype=f32, device=device)
        self.y = torch.zeros((1, hidden // 32 * 36), dtype=u8, device=device)
        self.h = torch.zeros((n_used + 1, ffn), dtype=f32, device=device)   # row n_used: shared expert
        self.hq = torch.zeros((n_used + 1, ffn // 32 * 36), dtype=u8, device=device)   # q8_1 copy of h
        self.o = torch.zeros((n_used, hidden), dtype=f32, device=device)
        self.o_sh = torch.zeros((1, hidden), dtype=f32, device=device)
        self.ids = torch.zeros((n_layers, 1, n_used), dtype=i32, device=device)
        self.w = torch.zeros((n_layers, 1, n_used), dtype=f32, device=device)
        # ffn_norm weight of each layer (RMSNorm in front of its MoE block)
        self.norm = torch.empty((n_layers, hidden), dtype=f32, device=device).uniform_(0.5, 1.5, generator=gen)
        for ly in self.layers:
            ly.f_gu = make_fusion(gate=ly.gate, glu_op=GLU_SWIGLU, shared_up=ly.sh_up, shared_gate=ly.sh_gate,
                                  shared_dst=self.h[n_used:], shared_type=sh_type)
            ly.f_dn = make_fusion(shared_up=ly.sh_down, shared_dst=self.o_sh, shared_type=sh_type,
                                  shared_src1=self.h[n_used:], shared_stride_col_y=ffn)
            ly.f_dnq = make_fusion(shared_up=ly.sh_down, shared_type=sh_type, shared_src1=self.hq[n_used:],
                                   shared_stride_col_y=ffn // 32)
        self.graph = None

    @property
    def f32_rows(self):
        """Fused plan: the GLU rows reach the down launch as fp32 rows (q8_K dots, or the fp32 hand-off)."""
        return self.fused and (self.act == "q8_K" or self.hand_off == "f32")

    # Algorithmic bytes: unique expert matrices + shared expert + the activations
    # and outputs each launch of the plan reads or writes once.
    def gate_up_bytes(self):
        H, F, U = self.H, self.F, self.U
        w = U * 2 * row_bytes(self.wtype, H) * F + 2 * row_bytes(self.sh_type, H) * F
        if self.f32_rows:                              # x row + norm weight in, fp32 GLU rows out
            return w + 2 * H * 4 + (U + 1) * F * 4
        if self.fused:                                 # x row + norm weight in, GLU rows (fp32 + q8_1) out
            return w + 2 * H * 4 + (U + 1) * F * 4 + (U + 1 if self.shared_q8 else U) * F // 32 * 36
        return w + H // 32 * 36 + (U + 1) * F * 4      # q8_1 row in, GLU rows out

    def down_bytes(self, l=None):
        """Bytes of layer l's down launch (l None: the mean over the layers)."""
        if l is None:
            return sum(self.down_bytes(k) for k in range(self.L)) // self.L
        H, F, U = self.H, self.F, self.U
        w = U * row_bytes(self.down_types[l], F) * H + row_bytes(self.sh_type, F) * H
        if self.f32_rows:                              # fp32 GLU rows, residual, router weights in; x out
            return w + (U + 1) * F * 4 + 2 * H * 4 + U * 4
        if self.fused:                                 # q8_1 (+ fp32 shared) GLU rows, residual, router weights in; x out
            sh_in = F // 32 * 36 if self.shared_q8 else F * 4
            return w + U * F // 32 * 36 + sh_in + 2 * H * 4 + U * 4
        return w + (U + 1) * F * 4 + (U + 1) * H * 4   # GLU rows in, expert outputs out

    def combine_bytes(self):
        H, U = self.H, self.U
        return 0 if self.fused else (U + 1) * H * 4 + 2 * H * 4 + H * 4 + H // 32 * 36 + U * 4

    def bytes_per_token(self):
        return sum(self.gate_up_bytes() + self.down_bytes(l) + self.combine_bytes() for l in range(self.L))

    def _stream(self):
        return C.c_void_p(self.torch.cuda.current_stream().cuda_stream)

    def launch_gate_up(self, l, s=None):
        ly = self.layers[l]
        s = s or self._stream()
        H, F, U = self.H, self.F, self.U
        check(lib().ggml_hip_moe_mul_mat_vec_ex(0, ACT_Q8_1, C.byref(ly.t_up), None, C.byref(ly.f_gu),
                                                self.y.data_ptr(), self.ids[l].data_ptr(), self.h.data_ptr(),
                                                H, F, self.E, 1, 1, U, H // 32, U * F, H // 32, F, U, s), "gate_up")

    def launch_down(self, l, s=None):
        ly = self.layers[l]
        s = s or self._stream()
        H, F, U = self.H, self.F, self.U
        check(lib().ggml_hip_moe_mul_mat_vec_ex(0, ACT_F32, C.byref(ly.t_down), None, C.byref(ly.f_dn),
                                                self.h.data_ptr(), self.ids[l].data_ptr(), self.o.data_ptr(),
                                                F, H, self.E, 1, U, U, (U + 1) * F, U * H, F, H, U, s),
              "down")

    def launch_layer(self, l, s=None):
        s = s or self._stream()
        H, F, U = self.H, self.F, self.U
        self.launch_gate_up(l, s)
        self.launch_down(l, s)
        src, dst = (self.x, self.x_next) if l % 2 == 0 else (self.x_next, self.x)
        nxt = self.norm[(l + 1) % self.L]        # the next block's ffn_norm (layer 0's for the next token)
        check(lib().ggml_hip_moe_combine_q8_1(self.o.data_ptr(), H, self.w[l].data_ptr(), U, self.o_sh.data_ptr(), H,
                                              src.data_ptr() if self.residual else None, dst.data_ptr(),
                                              self.y.data_ptr(), H // 32, H, 1, 1, nxt.data_ptr(), self.eps, s),
              "combine")

    def launch_gate_up_norm(self, l, src, s=None):
        """Fused plan, launch 1 of layer l: gate/up GEMV on q8_1(RMSNorm(src) * norm[l])."""
        ly = self.layers[l]
        s = s or self._stream()
        H, F, U = self.H, self.F, self.U
        nb = F // 32
        if self.act == "q8_K":
            check(lib().ggml_hip_moe_ffn_gate_up_norm_ex(0, ACT_Q8_K, C.byref(ly.t_up), None, C.byref(ly.f_gu),
                                                         src.data_ptr(), self.norm[l].data_ptr(), self.eps,
                                                         self.ids[l].data_ptr(), self.h.data_ptr(), H, F, self.E, 1, U,
                                                         H, U * F, F, U, None, 0, None, 0, 0, None, 0, s),
                  "gate_up_norm q8_K")
            return
        q8 = not self.f32_rows                         # q8_1 copies of the GLU rows
        check(lib().ggml_hip_moe_ffn_gate_up_norm(0, C.byref(ly.t_up), None, C.byref(ly.f_gu), src.data_ptr(),
                                                  self.norm[l].data_ptr(), self.eps, self.ids[l].data_ptr(),
                                                  self.h.data_ptr(), H, F, self.E, 1, U, H, U * F, F, U, None, 0,
                                                  self.hq.data_ptr() if q8 else None, (U + 1) * nb, nb,
                                                  self.hq[U:].data_ptr() if q8 and self.shared_q8 else None,
                                                  (U + 1) * nb, s),
              "gate_up_norm")

    def launch_down_combine(self, l, src, dst, s=None):
        """Fused plan, launch 2 of layer l: dst = src + shared + sum_j w_j * down_j(h_j)."""
        ly = self.layers[l]
        s = s or self._stream()
        H, F, U = self.H, self.F, self.U
        nb = F // 32
        if self.act == "q8_K":                         # fp32 GLU rows, quantized to q8_K by each wave
            check(lib().ggml_hip_moe_ffn_down_combine(0, ACT_F32 | ACT_DOT_Q8_K, C.byref(ly.t_down), C.byref(ly.f_dn),
                                                      self.h.data_ptr(), self.ids[l].data_ptr(), self.w[l].data_ptr(),
                                                      src.data_ptr() if self.residual else None, dst.data_ptr(),
                                                      F, H, self.E, 1, U, (U + 1) * F, F, H, U, s),
                  "down_combine q8_K")
            return
        if self.f32_rows:                              # fp32 GLU rows, quantized to q8_1 by each wave
            check(lib().ggml_hip_moe_ffn_down_combine(0, ACT_F32, C.byref(ly.t_down), C.byref(ly.f_dn),
                                                      self.h.data_ptr(), self.ids[l].data_ptr(), self.w[l].data_ptr(),
                                                      src.data_ptr() if self.residual else None, dst.data_ptr(),
                                                      F, H, self.E, 1, U, (U + 1) * F, F, H, U, s),
                  "down_combine f32 rows")
            return
        act = ACT_Q8_1 if self.shared_q8 else ACT_Q8_1 | ACT_SHARED_F32
        check(lib().ggml_hip_moe_ffn_down_combine(0, act, C.byref(ly.t_down),
                                                  C.byref(ly.f_dnq if self.shared_q8 else ly.f_dn),
                                                  self.hq.data_ptr(), self.ids[l].data_ptr(), self.w[l].data_ptr(),
                                                  src.data_ptr() if self.residual else None, dst.data_ptr(),
                                                  F, H, self.E, 1, U, (U + 1) * nb, nb, H, U, s),
              "down_combine")

    def launch_token(self):
        """One token through every layer; the token's input and output are in self.x."""
        s = self._stream()
        if self.fused:
            for l in range(self.L):
                src, dst = (self.x, self.x_next) if l % 2 == 0 else (self.x_next, self.x)
                self.launch_gate_up_norm(l, src, s)
                self.launch_down_combine(l, src, dst, s)
            if self.L % 2 == 1:
                self.x.copy_(self.x_next)
            return
        # ffn_norm of the first MoE block and q8_1 of its output
        check(lib().ggml_hip_moe_combine_q8_1(None, 0, None, 0, None, 0, self.x.data_ptr(), None, self.y.data_ptr(),
                                              self.H // 32, self.H, 1, 1, self.norm[0].data_ptr(), self.eps, s),
              "norm x")
        for l in range(self.L):
            self.launch_layer(l, s)
        if self.L % 2 == 1:
            self.x.copy_(self.x_next)

    def set_routing(self, ids, w):
        """ids: int32 [L, n_used], w: fp32 [L, n_used] (device or host tensors)."""
        self.ids.view(self.L, self.U).copy_(ids, non_blocking=True)
        self.w.view(self.L, self.U).copy_(w, non_blocking=True)

    def capture(self):
        torch = self.torch
        self.launch_token()                      # first use builds every device table
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.launch_token()
        torch.cuda.current_stream().wait_stream(s)
        self.graph = g
        return g

    def replay(self):
        self.graph.replay()


def make_routing(n_tokens, n_layers, n_experts, n_used, seed=0):
    """Uniform top-n_used ids without replacement and softmax router weights over N(0,1) logits."""
    rng = np.random.default_rng(seed)
    ids = np.empty((n_tokens, n_layers, n_used), np.int32)
    for t in range(n_tokens):
        for l in range(n_layers):
            ids[t, l] = rng.choice(n_experts, size=n_used, replace=False)
    logits = rng.standard_normal((n_tokens, n_layers, n_used)).astype(np.float32)
    w = np.exp(logits - logits.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    return ids, w.astype(np.float32)
