#!/usr/bin/env python3
"""Benchmark of the fused elementwise / row-reduction layer path on one MI355X.

A step is one launch of the path's kernel over one batch of the BASELINE
configuration (`--workload`, default configs[1]: residual add + RMSNorm on
fp32 [4096 x 4096]).  Inputs are resident in HBM before the timed region;
several buffer sets are rotated so the footprint of consecutive steps exceeds
the 256 MiB Infinity Cache and every step streams from HBM.  Before the W
warm-up steps the op runs for 0.25 s of GPU time so the clocks leave the
idle state the host uploads left them in.  Time is taken with HIP events
recorded on the context's stream around exactly K steps, between two stream
synchronisations.

Prints ONE compact JSON line on stdout (under 4 KB; progress goes to
stderr).  Besides the headline workload, `ops` summarises every op of
configs[0..4] measured the same way as [us per launch, GB/s, fraction of
peak, parity pass, HBM traffic over algorithmic bytes]; the full per-op
records go to `--full-out`.  `cpu_baseline` times the reference's own
CPU code (compiled from the reference sources into oracle/_ref) on the host, single-threaded as the
reference ops are.  The same leg checks each op: one more launch on freshly
uploaded inputs, compared with the CPU path's output on those inputs
(`parity`: max |d|, max relative error, bit-exactness, pass under the
path's tolerance).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "mimir-framework_amd"))

import mimir_hip as M  # noqa: E402
from mimir_hip import datagen as G  # noqa: E402

METRIC = "achieved HBM GB/s (% of MI355X peak) + rows/s per fused layer op vs host CPU"
PEAK_GBS = 8000.0  # MI355X HBM3E
PEAK_F32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix-core peak
MALL_BYTES = 256 << 20
MIN_FOOTPRINT = 5 * MALL_BYTES  # rotate buffer sets until one pass covers 1.25 GiB
MAX_SETS = 32
STDOUT_LIMIT = 4000  # the JSON line on stdout stays well inside the driver's tail


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class OpBench:
    """One op of one configuration: its inputs on the device (nsets copies)
    and a closure that launches it on set i."""

    def __init__(self, key, config, desc, kernel, nbytes, rows, row_unit, make, outputs=None, flops=None):
        self.key, self.config, self.desc, self.kernel = key, config, desc, kernel
        self.nbytes, self.rows, self.row_unit = nbytes, rows, row_unit
        # Matrix-core ops: algorithmic flops per launch (the roofline is the
        # fp32 MFMA peak, not HBM).
        self.flops = flops
        self.make = make  # make(ctx, nsets) -> (step(i), buffers)
        # outputs(buffers) -> {name: DeviceArray or ndarray}: what one launch
        # on set 0 produced, for the parity check of the cpu_baseline leg
        self.outputs = outputs

    def nsets(self):
        return max(2, min(MAX_SETS, math.ceil(MIN_FOOTPRINT / self.nbytes)))


def _replicate(ctx, host_arrays, nsets):
    """Upload each array once and device-copy it into nsets buffers."""
    sets = []
    for s in range(nsets):
        bufs = []
        for a in host_arrays:
            d = ctx.empty(a.shape, a.dtype)
            if s == 0:
                ctx.upload(d, a)
            else:
                ctx.copy(d, sets[0][len(bufs)], a.nbytes)
            bufs.append(d)
        sets.append(bufs)
    return sets


def small_stack(blocks=4, seq=128, e=256, heads=4):
    """A small transformer stack for the launch-bound runtime measurement:
    `blocks` pre-norm half-blocks (LayerNorm -> SelfAttention -> Add ->
    LayerNorm -> GELU) on [seq x e], 5 layers each, reading "inp" and
    leaving "x".  Returns (layers, float inputs)."""
    r = G.rng(5, 0)
    layers, cur = [], "inp"
    for b in range(blocks):
        g = np.concatenate([1 + 0.05 * r.standard_normal(e), 0.05 * r.standard_normal(e)]).astype(np.float32)
        w = (r.standard_normal(4 * e * e) / np.sqrt(e)).astype(np.float32)
        out = "x" if b == blocks - 1 else f"h{b}"
        layers += [dict(name=f"ln{b}", type="LayerNorm", inputs=[cur], output=f"n{b}", in_features=e, weights=g),
                   dict(name=f"attn{b}", type="SelfAttention", inputs=[f"n{b}"], output=f"a{b}", seq_len=seq,
                        embed_dim=e, num_heads=heads, causal=True, weights=w),
                   dict(name=f"res{b}", type="Add", inputs=[f"a{b}", cur], output=f"r{b}"),
                   dict(name=f"ln2_{b}", type="LayerNorm", inputs=[f"r{b}"], output=f"m{b}", in_features=e,
                        weights=g),
                   dict(name=f"act{b}", type="GELU", inputs=[f"m{b}"], output=out)]
        cur = out
    return layers, {"inp": r.standard_normal(seq * e).astype(np.float32)}


def block_layers():
    """A residual block's chain of the path's layers at the configs[4] shape,
    routed by name.  The result is named "x", the tensor
    Model::forwardPassNamed returns."""
    _, g, b, _ = G.cfg4_layernorm(rows=1)
    return [dict(name="res_add", type="Add", inputs=["inp", "res"], output="h"),
            dict(name="ln", type="LayerNorm", inputs=["h"], output="n", in_features=4096, eps=1e-5,
                 weights=np.concatenate([g, b])),
            dict(name="act", type="GELU", inputs=["n"], output="g"),
            dict(name="gate", type="Multiply", inputs=["g", "gate"], output="m"),
            dict(name="silu", type="SiLU", inputs=["m"], output="x")]


def attention_flops(batch, heads, q_len, kv_len, head_dim, causal):
    """Algorithmic flops of the attention core: 2*head_dim for each visible
    (query, key) pair in QK^T and again in PV (the softmax's exponentials are
    not counted).  Causal: query i sees min(i + 1, kv_len) keys."""
    if causal:
        i = np.arange(q_len)
        pairs = int(np.minimum(i + 1, kv_len).sum())
    else:
        pairs = q_len * kv_len
    return 4 * head_dim * pairs * batch * heads


def attention_bwd_flops(batch, heads, q_len, kv_len, head_dim, causal):
    """Algorithmic flops of the attention core's backward: the five products
    of backward_self_attention (S = QK^T, dP = dO V^T, dV = P^T dO,
    dQ = dS K, dK = dS^T Q) over the visible (query, key) pairs, 2*head_dim
    each (the masked pairs contribute nothing)."""
    return attention_flops(batch, heads, q_len, kv_len, head_dim, causal) // 4 * 10


def build_ops(rows_override=None):
    """Every op of the sweep.  rows_override (bench --rows) changes the row
    count of the configs[1] add + RMSNorm and configs[4] LayerNorm ops only,
    for size sweeps that separate a kernel's per-launch cost from its
    streaming rate; the default lines use the configs' own sizes."""
    ops = []
    f4 = 4

    def ln_op(key, cfg, gen, rows, cols):
        def make(ctx, nsets):
            x, g, b, eps = gen()
            gb = _replicate(ctx, [g, b], 1)[0]
            sets = _replicate(ctx, [x, np.empty_like(x)], nsets)
            return (lambda i: ctx.layernorm(sets[i][0], gb[0], gb[1], sets[i][1], rows, cols, eps)), sets + [gb]
        return OpBench(key, cfg, f"LayerNorm fp32 [{rows}x{cols}]", "norm_rows_vec<Layer>",
                       2 * rows * cols * f4 + 2 * cols * f4, rows, "rows", make, lambda s: {"y": s[0][1]})

    ops.append(ln_op("cfg0_layernorm", 0, G.cfg0_layernorm, 256, 512))

    r1 = rows_override or 4096

    def make_cfg1(ctx, nsets):
        x, r, w, eps = G.cfg1_add_rmsnorm(rows=r1)
        wd = _replicate(ctx, [w], 1)[0][0]
        sets = _replicate(ctx, [x, r, np.empty_like(x)], nsets)
        return (lambda i: ctx.add_rmsnorm(sets[i][0], sets[i][1], sets[i][1], wd, sets[i][2], r1, 4096,
                                          eps)), sets + [[wd]]
    ops.append(OpBench("cfg1_add_rmsnorm", 1, f"residual add + RMSNorm fp32 x,r [{r1}x4096] -> y, residual'",
                       "norm_rows_vec<AddRms>", 4 * r1 * 4096 * f4 + 4096 * f4, r1, "rows", make_cfg1,
                       lambda s: {"y": s[0][2], "residual": s[0][1]}))

    def make_cfg2(ctx, nsets):
        s = G.cfg2_softmax().reshape(-1, 1024)
        sets = _replicate(ctx, [s, np.empty_like(s)], nsets)
        del s
        return (lambda i: ctx.softmax(sets[i][0], sets[i][1], 262144, 1024, M.SOFTMAX_DIV_EPS)), sets
    ops.append(OpBench("cfg2_softmax", 2, "causal row softmax fp32 [8x32x1024x1024]", "softmax_rows_vec",
                       2 * 262144 * 1024 * f4, 262144, "rows", make_cfg2, lambda s: {"y": s[0][1]}))

    # The attention core at configs[2]'s shape (8 sequences x 32 heads x 1024
    # tokens, causal), head_dim 128, on a fused [8192 x 12288] QKV buffer: the
    # softmax of configs[2] fused between QK^T and PV (matrix-core bound).
    ab, al, ah, ad = 8, 1024, 32, 128
    aw = ah * ad

    def make_attention(ctx, nsets):
        qkv = G.attention_qkv(ab, al, ah, ad)
        sets = _replicate(ctx, [qkv, np.empty((ab * al, aw), np.float32)], nsets)
        del qkv
        return (lambda i: ctx.attention(sets[i][0], sets[i][0].offset(aw), sets[i][0].offset(2 * aw), sets[i][1],
                                        ab, al, al, ah, ad, True, ld_q=3 * aw, ld_kv=3 * aw)), sets
    ops.append(OpBench("f4_attention", 2,
                       f"fused causal attention core fp32 [{ab} seq x {ah} heads x {al} tokens, head_dim {ad}], "
                       f"fused QKV [{ab * al}x{3 * aw}] -> out [{ab * al}x{aw}]",
                       "attention_fwd_mfma<128>", 4 * ab * al * aw * f4, ab * ah * al, "query rows",
                       make_attention, lambda s: {"out": s[0][1]},
                       flops=attention_flops(ab, ah, al, al, ad, True)))

    def make_attention_bwd(ctx, nsets):
        qkv = G.attention_qkv(ab, al, ah, ad)
        sets = _replicate(ctx, [qkv, G.attention_dout(ab, al, ah, ad), np.empty_like(qkv)], nsets)
        del qkv

        def step(i):
            x, do, g = sets[i]
            ctx.attention_bwd(x, x.offset(aw), x.offset(2 * aw), do, g, g.offset(aw), g.offset(2 * aw), ab, al, al,
                              ah, ad, True, ld_q=3 * aw, ld_kv=3 * aw, ld_dout=aw, ld_dq=3 * aw, ld_dkv=3 * aw)
        return step, sets
    ops.append(OpBench("f4_attention_bwd", 2,
                       f"attention core backward fp32 [{ab} seq x {ah} heads x {al} tokens, head_dim {ad}, causal]: "
                       f"QKV [{ab * al}x{3 * aw}] + dout [{ab * al}x{aw}] -> dQKV [{ab * al}x{3 * aw}]",
                       "hipBLASLt sgemm (S, dP, dQ, dV, dK on two causal blocks each) + attn_probs_dsoftmax_kernel<16> + "
                       "heads_to_rows_kernel",
                       7 * ab * al * aw * f4, ab * ah * al, "query rows", make_attention_bwd,
                       lambda s: {"dqkv": s[0][2]}, flops=attention_bwd_flops(ab, ah, al, al, ad, True)))

    def make_cfg3a(ctx, nsets):
        table, ids = G.cfg3_gather()
        sets = _replicate(ctx, [table, ids, np.empty((ids.size, 4096), np.float32)], nsets)
        del table
        return (lambda i: ctx.embedding(sets[i][1], 32768, sets[i][0], 32000 * 4096, 32000, 4096, -1,
                                        sets[i][2])), sets
    ops.append(OpBench("cfg3_gather", 3, "token-embedding gather table [32000x4096] ids int32 [16x2048]",
                       "embed_vec", 32768 * 4 + 2 * 32768 * 4096 * f4, 32768, "token rows", make_cfg3a,
                       lambda s: {"y": s[0][2]}))

    def make_cfg3b(ctx, nsets):
        q, k, theta = G.cfg3_rope()
        c, s = M.rope_table(2048, 128, theta)
        cs = _replicate(ctx, [c, s], 1)[0]
        sets = _replicate(ctx, [q, k], nsets)
        del q, k
        return (lambda i: ctx.rope(sets[i][0], sets[i][0], 32, sets[i][1], sets[i][1], 32, 16, 2048, 128, 0,
                                   cs[0], cs[1], 2048)), sets + [cs]
    ops.append(OpBench("cfg3_rope", 3, "RoPE q,k [16x2048x32x128] in place, one launch", "rope_vec",
                       2 * 2 * 16 * 2048 * 32 * 128 * f4, 2 * 16 * 2048 * 32, "head rows", make_cfg3b,
                       lambda s: {"q": s[0][0], "k": s[0][1]}))

    r4 = rows_override or 8192
    ops.append(ln_op("cfg4_layernorm", 4, lambda: G.cfg4_layernorm(rows=r4), r4, 4096))

    def make_gelu(ctx, nsets):
        a = G.cfg4_gelu()
        sets = _replicate(ctx, [a, np.empty_like(a)], nsets)
        return (lambda i: ctx.gelu(sets[i][0], sets[i][1], a.size)), sets
    ops.append(OpBench("cfg4_gelu", 4, "tanh-GELU fp32 [8192x11008]", "unary_vec<Gelu>",
                       2 * 8192 * 11008 * f4, 8192, "rows", make_gelu, lambda s: {"y": s[0][1]}))

    def make_swiglu(ctx, nsets):
        g, u = G.cfg4_swiglu()
        sets = _replicate(ctx, [g, u, np.empty_like(g)], nsets)
        return (lambda i: ctx.silu_mul(sets[i][0], sets[i][1], sets[i][2], g.size)), sets
    ops.append(OpBench("cfg4_silu_mul", 4, "SiLU-gated product silu(gate)*up fp32 [8192x11008]",
                       "binary_vec<SiluMul>", 3 * 8192 * 11008 * f4, 8192, "rows", make_swiglu,
                       lambda s: {"y": s[0][2]}))

    def make_add(ctx, nsets):
        a, b = G.cfg4_add()
        sets = _replicate(ctx, [a, b, np.empty_like(a)], nsets)
        return (lambda i: ctx.add(sets[i][0], a.size, sets[i][1], b.size, sets[i][2])), sets
    ops.append(OpBench("cfg4_add", 4, "residual add fp32 [8192x4096]", "binary_vec<Add>",
                       3 * 8192 * 4096 * f4, 8192, "rows", make_add, lambda s: {"y": s[0][2]}))

    # The reference's Softmax and RMSNorm layers, and LayerNorm with
    # in_features unset, normalise their whole input as one row
    # (LayerOps.hpp:276, :325-361; LayerOpsExt.hpp:345-378): the configs[4]
    # activation [8192x4096] is then one row of 2^25 floats, cut into chunks
    # over the whole GPU (partial, combine, apply).
    def make_whole(kind):
        def make(ctx, nsets):
            x, _, _, eps = G.cfg4_layernorm()
            w = G.cfg4_layernorm(rows=1)[1]  # an RMSNorm weight block of in_features = 4096
            wd = _replicate(ctx, [w], 1)[0][0]
            sets = _replicate(ctx, [x, np.empty_like(x)], nsets)
            n = x.size
            del x
            if kind == "softmax":
                return (lambda i: ctx.softmax(sets[i][0], sets[i][1], 1, n, M.SOFTMAX_MUL_INV)), sets + [[wd]]
            if kind == "rmsnorm":
                return (lambda i: ctx.rmsnorm(sets[i][0], wd, w.size, sets[i][1], 1, n, eps)), sets + [[wd]]
            return (lambda i: ctx.layernorm(sets[i][0], None, None, sets[i][1], 1, n, eps)), sets + [[wd]]
        return make
    for kind, desc, kern, extra in (
            ("softmax", "Softmax layer over the configs[4] activation as one row of 2^25 fp32",
             "lr_partial<Softmax> + lr_combine + lr_apply", 0),
            ("rmsnorm", "RMSNorm layer (weights 4096) over the configs[4] activation as one row of 2^25 fp32",
             "lr_partial<SumSq> + lr_combine + lr_apply", 4096 * f4),
            ("layernorm", "LayerNorm layer (in_features unset, no weight block) over the configs[4] activation "
             "as one row of 2^25 fp32", "lr_partial<Chan> + lr_combine + lr_apply", 0)):
        ops.append(OpBench(f"cfg4_{kind}_whole", 4, desc, kern, 2 * 8192 * 4096 * f4 + extra, 1, "rows",
                           make_whole(kind), lambda s: {"y": s[0][1]}))

    # Backward of the same ops (Model::backwardPass branches, Model.cpp:7305-9153)
    # at the configs[3] / configs[4] shapes.
    def make_lnb(ctx, nsets):
        x, g, b, eps = G.cfg4_layernorm()
        dy = G.cfg4_grad(x.shape, 8)
        pd = _replicate(ctx, [g, np.zeros_like(g), np.zeros_like(b)], 1)[0]
        sets = _replicate(ctx, [x, dy, np.empty_like(x)], nsets)
        return (lambda i: ctx.layernorm_bwd(sets[i][0], sets[i][1], pd[0], sets[i][2], pd[1], pd[2], 8192, 4096,
                                            eps)), sets + [pd]
    ops.append(OpBench("cfg4_layernorm_bwd", 4, "LayerNorm backward fp32 [8192x4096]: dx, dgamma, dbeta",
                       "ln_bwd_vec + slot sums", 3 * 8192 * 4096 * f4 + 5 * 4096 * f4, 8192, "rows", make_lnb,
                       lambda s: {"dx": s[0][2], "dgamma": s[-1][1], "dbeta": s[-1][2]}))

    def make_act_bwd(fn_name):
        def make(ctx, nsets):
            a = G.cfg4_gelu()
            dy = G.cfg4_grad(a.shape, 9)
            sets = _replicate(ctx, [a, dy, np.empty_like(a)], nsets)
            fn = getattr(ctx, fn_name)
            return (lambda i: fn(sets[i][0], sets[i][1], sets[i][2], a.size)), sets
        return make
    ops.append(OpBench("cfg4_gelu_bwd", 4, "GELU backward fp32 [8192x11008]", "dact_vec<DGelu>",
                       3 * 8192 * 11008 * f4, 8192, "rows", make_act_bwd("gelu_bwd"), lambda s: {"dx": s[0][2]}))
    ops.append(OpBench("cfg4_silu_bwd", 4, "SiLU backward fp32 [8192x11008]", "dact_vec<DSilu>",
                       3 * 8192 * 11008 * f4, 8192, "rows", make_act_bwd("silu_bwd"), lambda s: {"dx": s[0][2]}))

    def make_mulb(ctx, nsets):
        g, u = G.cfg4_swiglu()
        dy = G.cfg4_grad(g.shape, 10)
        sets = _replicate(ctx, [g, u, dy, np.empty_like(g), np.empty_like(g)], nsets)
        return (lambda i: ctx.mul_bwd(sets[i][0], sets[i][1], sets[i][2], sets[i][3], sets[i][4], g.size)), sets
    ops.append(OpBench("cfg4_mul_bwd", 4, "Multiply backward fp32 [8192x11008]: da, db", "mul_bwd_vec",
                       5 * 8192 * 11008 * f4, 8192, "rows", make_mulb, lambda s: {"da": s[0][3], "db": s[0][4]}))

    def make_addb(ctx, nsets):
        a, _ = G.cfg4_add()
        sets = _replicate(ctx, [a, np.empty_like(a), np.empty_like(a)], nsets)
        return (lambda i: ctx.add_bwd(sets[i][0], a.size, a.size, sets[i][1], sets[i][2])), sets
    ops.append(OpBench("cfg4_add_bwd", 4, "residual Add backward fp32 [8192x4096]: da, db", "add_bwd_vec",
                       3 * 8192 * 4096 * f4, 8192, "rows", make_addb, lambda s: {"da": s[0][1], "db": s[0][2]}))

    # Embedding backward on the configs[3] ids (uniform), and on ids as text
    # has them (Zipf, s = 1: the most frequent id is ~9% of the tokens).
    def make_embb(ids_fn):
        def make(ctx, nsets):
            ids = ids_fn()
            dy = G.cfg3_embedding_grad()
            gt = _replicate(ctx, [np.zeros(32000 * 4096, np.float32)], 1)[0][0]
            sets = _replicate(ctx, [ids, dy], nsets)
            return (lambda i: ctx.embedding_bwd(sets[i][0], ids.size, sets[i][1], gt, 32000 * 4096, 32000, 4096,
                                                -1)), sets + [[gt]]
        return make
    for key, ids_fn, what in (("cfg3_embedding_bwd", G.cfg3_ids, "ids int32 [16x2048]"),
                              ("cfg3_embedding_bwd_zipf", G.cfg3_ids_zipf, "Zipf(1.0) ids int32 [16x2048]")):
        ids_ = ids_fn()
        u = int(np.unique(ids_).size)
        top = int(np.bincount(ids_.ravel()).max())
        ops.append(OpBench(key, 3, f"Embedding backward (scatter-add) {what} -> table grad [32000x4096], "
                           f"{u} distinct ids, longest run {top}",
                           "counting sort (embed_sort_count / _offsets / _scatter) + embed_bwd_rows_seg (runs, "
                           "segment partials, long-run list) + embed_bwd_seg_combine",
                           32768 * 4 + 32768 * 4096 * f4 + 2 * u * 4096 * f4, 32768, "token rows", make_embb(ids_fn),
                           lambda s: {"grad": s[-1][0]}))

    # The device-resident runtime (mimir_store_run): a residual block's chain
    # of the path's layers at the configs[4] shape, routed by name as
    # Model::forwardPassNamed does; a step is one run of the five layers.
    class _Owned:
        def __init__(self, *objs):
            self.objs = objs

        def free(self):
            for o in self.objs:
                o.close()

    def make_block(ctx, nsets):
        x, res = G.cfg4_add()
        gate = G.cfg4_grad((8192, 4096), 11)
        layers = block_layers()
        graph = M.DeviceGraph(ctx, layers)
        store = M.Store(ctx)
        store.set_inputs({"inp": x, "res": res, "gate": gate}, {})
        store.run(graph)  # fills the buffer pool: later runs allocate nothing
        return (lambda i: store.run(graph)), [[_Owned(store, graph)]]
    blk = OpBench("cfg4_runtime_block", 4,
                  "device-resident runtime: Add -> LayerNorm -> GELU -> Multiply -> SiLU on [8192x4096], routed by name",
                  "mimir_store_run (5 kernels)", 12 * 8192 * 4096 * f4 + 2 * 4096 * f4, 8192, "rows", make_block,
                  lambda s: {"x": s[0][0].objs[0].get("x")})
    blk.nsets = lambda: 1
    ops.append(blk)

    # The same block with the runtime's fusion on (mimir_store_set_fusion):
    # Add -> LayerNorm -> GELU -> Multiply -> SiLU run as one kernel (the
    # LayerNorm with an add prologue and an elementwise epilogue), so the
    # block moves 4 streams of [8192x4096] instead of 12: inp, res and gate
    # in, x out.
    def make_block_fused(ctx, nsets):
        x, res = G.cfg4_add()
        gate = G.cfg4_grad((8192, 4096), 11)
        graph = M.DeviceGraph(ctx, block_layers())
        store = M.Store(ctx)
        store.set_fusion(True)
        store.set_inputs({"inp": x, "res": res, "gate": gate}, {})
        store.run(graph)
        return (lambda i: store.run(graph)), [[_Owned(store, graph)]]
    bf = OpBench("cfg4_runtime_block_fused", 4,
                 "the same block with the runtime's fusion: the five layers as one kernel on [8192x4096]",
                 "norm_rows_vec<AddLayer, 512, 2, 512, epilogue>", 4 * 8192 * 4096 * f4 + 2 * 4096 * f4,
                 8192, "rows", make_block_fused, lambda s: {"x": s[0][0].objs[0].get("x")})
    bf.nsets = lambda: 1
    ops.append(bf)

    # One device-resident training step of the same block: forwardPassNamed
    # (training=true) then backwardPass with the loss gradient already in HBM
    # (mimir_store_run_training + mimir_store_backward_dev).  Streams of
    # [8192x4096]: forward 12; backward: loss-gradient copy 2, SiLU 3,
    # Multiply 5, GELU 3, LayerNorm 3 (+ gamma, dgamma, dbeta), Add 3.
    def make_block_train(ctx, nsets):
        x, res = G.cfg4_add()
        gate = G.cfg4_grad((8192, 4096), 11)
        graph = M.DeviceGraph(ctx, block_layers())
        store = M.Store(ctx)
        store.set_inputs({"inp": x, "res": res, "gate": gate}, {})
        lg = ctx.to_device(G.cfg4_grad((8192, 4096), 12))

        def step(i):
            store.run_training(graph)
            store.backward(graph, lg)
        step(0)  # fills the buffer pool: later steps allocate nothing
        return step, [[_Owned(store, graph), lg]]
    trn = OpBench("cfg4_runtime_block_train", 4,
                  "device-resident training step of the same block on [8192x4096]: forward (training) + backward",
                  "mimir_store_run_training + mimir_store_backward_dev (12 kernels)",
                  31 * 8192 * 4096 * f4 + 7 * 4096 * f4, 8192, "rows", make_block_train)
    trn.nsets = lambda: 1
    ops.append(trn)

    # Launch-bound: the small stack through the runtime with its fusion on
    # (per block: LayerNorm, the attention layer's 2 GEMMs + core, then Add ->
    # LayerNorm -> GELU as one kernel: 20 kernels), eager and as one captured
    # graph replayed (mimir_store_capture / _graph_launch).
    def make_stack(captured):
        def make(ctx, nsets):
            layers, fin = small_stack()
            graph = M.DeviceGraph(ctx, layers)
            store = M.Store(ctx)
            store.set_fusion(True)
            if captured:
                sg = store.capture(graph, fin, {})
                return (lambda i: sg.launch()), [[_Owned(sg, store, graph)]]
            store.set_inputs(fin, {})
            store.run(graph)  # fills the pool, the scratch and the library workspace
            return (lambda i: store.run(graph)), [[_Owned(store, graph)]]
        return make
    sl, _ = small_stack()
    for key, captured in (("f1_stack_eager", False), ("f1_stack_graph", True)):
        op = OpBench(key, -1, f"runtime forward of a small transformer stack ({len(sl)} layers, [128x256], 4 "
                     f"causal attention blocks, fusion on), "
                     f"{'one captured graph launch' if captured else 'eager launches'}",
                     "mimir_store_graph_launch" if captured else "mimir_store_run", 128 * 256 * f4, 128, "rows",
                     make_stack(captured))
        op.nsets = lambda: 1
        op.bound = "launch"
        ops.append(op)

    # Calibration: a plain streaming copy of 512 MiB (mimir_copy), the
    # practical HBM ceiling and the yardstick for the FETCH/WRITE counters.
    def make_copy(ctx, nsets):
        n = 128 << 20
        sets = [[ctx.empty(n), ctx.empty(n)] for _ in range(nsets)]
        return (lambda i: ctx.copy(sets[i][1], sets[i][0], n * 4)), sets
    ops.append(OpBench("calib_copy", -1, "streaming copy 512 MiB (mimir_copy)", "copy16_kernel",
                       2 * (128 << 20) * f4, 128 << 20, "floats", make_copy))
    return ops


def spin_up(ctx, step, nsets, seconds):
    """Run the op until `seconds` of GPU time have passed: the GPU lowers its
    clocks while the host uploads inputs, and a few launches do not bring
    them back (the first tens of ms run ~4% slower)."""
    e0, e1 = ctx.event(), ctx.event()
    done, n = 0.0, 0
    try:
        while done < seconds * 1e3:
            e0.record()
            for i in range(16):
                step((n + i) % nsets)
            e1.record()
            done += e0.elapsed_ms(e1)
            n += 16
    finally:
        e0.close()
        e1.close()
    return n


def time_op(ctx, op, steps, warmup, spin_s=0.25):
    nsets = op.nsets()
    step, sets = op.make(ctx, nsets)
    try:
        spin_up(ctx, step, nsets, spin_s)
        for i in range(warmup):
            step(i % nsets)
        ctx.sync()
        e0, e1 = ctx.event(), ctx.event()
        e0.record()
        for i in range(steps):
            step(i % nsets)
        e1.record()
        ctx.sync()
        ms = e0.elapsed_ms(e1)
        e0.close()
        e1.close()
    finally:
        for bufs in sets:
            for b in bufs:
                b.free()
    us = ms * 1e3 / steps
    gbs = op.nbytes / (us * 1e-6) / 1e9
    rec = {
        "op": op.key, "config": op.config, "desc": op.desc, "kernel": op.kernel,
        "algorithmic_bytes": op.nbytes, "us_per_launch": round(us, 3), "GB_s": round(gbs, 1),
        "frac_of_peak": round(gbs / PEAK_GBS, 4), "rows_per_s": round(op.rows / (us * 1e-6), 1),
        "row_unit": op.row_unit, "launches": steps, "buffer_sets": nsets,
        "footprint_MiB": round(nsets * op.nbytes / 2**20, 1),
    }
    if getattr(op, "bound", None) == "launch":
        rec.update({"bound": "launch", "GB_s": None, "frac_of_peak": None})
    elif op.flops:
        tf = op.flops / (us * 1e-6) / 1e12
        rec.update({"bound": "mfma", "algorithmic_flops": op.flops, "TFLOP_s": round(tf, 2),
                    "frac_of_peak": round(tf / PEAK_F32_MFMA_TFLOPS, 4), "peak": PEAK_F32_MFMA_TFLOPS,
                    "peak_unit": "TFLOP/s (dense fp32 MFMA)", "frac_of_hbm_peak": round(gbs / PEAK_GBS, 4)})
    return rec


def same_bytes_copy(ctx, nbytes, steps, warmup, cache):
    """A plain streaming copy moving `nbytes` per launch (half read, half
    written), timed like the ops: the practical ceiling of a stream that size.
    Cached by size (several ops move the same bytes)."""
    n_copy = (nbytes // 8) // 4 * 4
    if n_copy not in cache:
        def make(ctx, nsets):
            sets = [[ctx.empty(n_copy), ctx.empty(n_copy)] for _ in range(nsets)]
            return (lambda i: ctx.copy(sets[i][1], sets[i][0], n_copy * 4)), sets
        cache[n_copy] = time_op(ctx, OpBench("copy_same_bytes", -1, "copy of the op's bytes", "copy16_kernel",
                                             8 * n_copy, n_copy, "floats", make), steps, warmup)
    return cache[n_copy]


def time_queued(ctx, op, launches=200):
    """Device-side time per launch of a small op: the launches are enqueued
    behind ~3 ms of copies, so the GPU runs them back to back with the host
    already out of the way; events bracket the launches alone.  (Timed one
    Python call at a time, an op this small measures the host's call rate.)"""
    nsets = op.nsets()
    step, sets = op.make(ctx, nsets)
    n = 64 << 20
    a, b = ctx.empty(n), ctx.empty(n)
    try:
        for i in range(8):
            step(i % nsets)
        ctx.sync()
        e0, e1 = ctx.event(), ctx.event()
        for _ in range(40):  # ~80 us each: the GPU stays busy while the host enqueues
            ctx.copy(b, a, n * 4)
        e0.record()
        for i in range(launches):
            step(i % nsets)
        e1.record()
        ctx.sync()
        us = e0.elapsed_ms(e1) * 1e3 / launches
        e0.close()
        e1.close()
    finally:
        a.free()
        b.free()
        for bufs in sets:
            for buf in bufs:
                buf.free()
    gbs = op.nbytes / (us * 1e-6) / 1e9
    return {"us_per_launch": round(us, 3), "GB_s": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4),
            "launches": launches, "method": "launches queued behind 40 copies of 256 MiB, events around the launches alone"}


# Ops too small to time one host call at a time: their sweep figure is the
# device-side one (time_queued), the host-driven one is kept beside it.
QUEUED_OPS = ("cfg0_layernorm",)


# ---------------------------------------------------------------------------
# CPU baseline leg: the reference's own code (oracle/_ref) or, for ops with no
# reference function, the C restatement (oracle/lib), single-threaded.
# ---------------------------------------------------------------------------

def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _whole_inputs(key):
    """(kind, flat x, RMSNorm weights, eps, reference fn, port fn, float64 exact fn) of a
    cfg4_*_whole op: the reference's own layer function, the C restatement,
    and the float64 value of the same formula."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    kind = key[len("cfg4_"):-len("_whole")]
    x, _, _, eps = G.cfg4_layernorm()
    x = x.ravel()
    w = G.cfg4_layernorm(rows=1)[1]
    if kind == "softmax":  # LayerOps::softmax_forward, the Model's Softmax layer
        ref = lambda: O.ref_softmax_forward(x)
        port = lambda: O.softmax_rows(x.reshape(1, -1), O.SOFTMAX_MUL_INV).ravel()

        def exact():
            e = np.exp(x.astype(np.float64) - float(x.max()))
            return e / e.sum()
    elif kind == "rmsnorm":  # LayerOpsExt rms_norm over the whole vector, weight i while i < 4096
        ref = lambda: O.ref_rms_norm_forward(x, w, eps=eps)
        port = lambda: O.rmsnorm_whole(x, w, eps)

        def exact():
            x64 = x.astype(np.float64)
            y = x64 / np.sqrt(np.mean(x64 * x64) + eps)
            y[:w.size] *= w
            return y
    else:  # LayerOps::layernorm_forward, normalized_size = the whole input, no weight block
        ref = lambda: O.ref_layernorm(x, 0, None, eps=eps)
        port = lambda: O.layernorm(x, x.size, None, None, eps)

        def exact():
            x64 = x.astype(np.float64)
            return (x64 - x64.mean()) / np.sqrt(x64.var() + eps)
    return kind, x, w, eps, ref, port, exact


def cpu_leg(which, reps):
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    have_ref = O.ref_available()
    out = {}

    def rec(key, seconds, nbytes, rows, kind, sample):
        gbs = nbytes / seconds / 1e9
        out[key] = {"value": round(gbs, 3), "unit": "GB/s", "seconds": round(seconds, 6),
                    "rows_per_s": round(rows / seconds, 1), "cores": 1, "kind": kind, "sample": sample}

    for key in which:
        log(f"cpu baseline: {key}")
        if key == "cfg1_add_rmsnorm":
            x, r, w, eps = G.cfg1_add_rmsnorm()
            nb = 4 * x.nbytes + w.nbytes
            if have_ref:
                t = O.ref_time_op(O.REF_T_ADD_RMSNORM, x, r, w, 4096, 4096, eps, reps)
                rec(key, t, nb, 4096, "reference",
                    "full configs[1] (4096x4096): LayerOps::add_forward then Normalization::rms_norm, "
                    f"median of {reps} calls")
            else:
                t = O.time_port(lambda: O.add_rmsnorm(x, r, w, eps), reps)
                rec(key, t, nb, 4096, "port", f"full configs[1], oracle add_rmsnorm, median of {reps}")
        elif key in ("cfg0_layernorm", "cfg4_layernorm"):
            x, g, b, eps = (G.cfg0_layernorm() if key == "cfg0_layernorm" else G.cfg4_layernorm())
            rows, cols = x.shape
            nb = 2 * x.nbytes + g.nbytes + b.nbytes
            if have_ref:
                t = O.ref_time_op(O.REF_T_LAYERNORM, x, None, np.concatenate([g, b]), rows, cols, eps, reps)
                rec(key, t, nb, rows, "reference", f"full [{rows}x{cols}] LayerOps::layernorm_forward")
            else:
                t = O.time_port(lambda: O.layernorm(x, cols, g, b, eps), reps)
                rec(key, t, nb, rows, "port", f"full [{rows}x{cols}] oracle layernorm")
        elif key == "cfg2_softmax":
            s = G.cfg2_softmax(batch=1, heads=4).reshape(-1, 1024)  # 1/64 of the rows
            nb = 2 * s.nbytes
            if have_ref:
                t = O.ref_time_op(O.REF_T_SOFTMAX, s, rows=s.shape[0], cols=1024, reps=reps)
                rec(key, t, nb, s.shape[0], "reference",
                    "4096 of 262144 causal rows (batch 1, heads 4) LayerOps::softmax_inplace")
            else:
                t = O.time_port(lambda: O.softmax_rows(s), reps)
                rec(key, t, nb, s.shape[0], "port", "4096 causal rows, oracle softmax_rows")
        elif key == "cfg3_gather":
            table, ids = G.cfg3_gather()
            nb = ids.nbytes + 2 * ids.size * 4096 * 4
            sys.path.insert(0, os.path.join(REPO, "oracle"))
            import model_ref as MR
            if MR.available():
                # The reference gather is inline in Model.cpp (:1152-1205): time it
                # through forwardPassNamed with one Embedding layer.
                layers = [dict(name="tok", type="Embedding", inputs=["ids"], output="x", vocab_size=32000,
                               embed_dim=4096, weights=table.ravel())]
                t = MR.time_forward_named(layers, {}, {"ids": ids.ravel()}, reps)
                rec(key, t, nb, ids.size, "reference",
                    "full configs[3]: Model::forwardPassNamed with one Embedding layer (the inline gather, "
                    "Model.cpp:1152-1205)")
            else:
                t = O.time_port(lambda: O.embedding(ids, table, 32000, 4096, -1), reps)
                rec(key, t, nb, ids.size, "port", "full configs[3] gather, oracle embedding_i32")
        elif key == "cfg3_rope":
            q, k, theta = G.cfg3_rope(batch=2)
            c, s = O.rope_table(2048, 128, theta)
            t = O.time_port(lambda: (O.rope(q, c, s), O.rope(k, c, s)), reps)
            rec(key, t, 2 * (q.nbytes + k.nbytes), 2 * 2 * 2048 * 32, "port",
                "batch 2 of 16, q and k, oracle rope (no reference RoPE exists)")
        elif key == "cfg4_gelu":
            a = G.cfg4_gelu(rows=512)
            if have_ref:
                t = O.ref_time_op(O.REF_T_GELU, a, reps=reps)
                rec(key, t, 2 * a.nbytes, 512, "reference", "512 of 8192 rows, LayerOps::gelu_forward")
            else:
                t = O.time_port(lambda: O.gelu(a), reps)
                rec(key, t, 2 * a.nbytes, 512, "port", "512 of 8192 rows, oracle gelu")
        elif key == "cfg4_silu_mul":
            g, u = G.cfg4_swiglu(rows=512)
            if have_ref:
                t = O.ref_time_op(O.REF_T_SILU_MUL, g, u, reps=reps)
                rec(key, t, 3 * g.nbytes, 512, "reference",
                    "512 of 8192 rows, multiply_forward(silu_forward(gate), up)")
            else:
                t = O.time_port(lambda: O.silu_mul(g, u), reps)
                rec(key, t, 3 * g.nbytes, 512, "port", "512 of 8192 rows, oracle silu_mul")
        elif key == "cfg4_add":
            a, b = G.cfg4_add()
            if have_ref:
                t = O.ref_time_op(O.REF_T_ADD, a, b, reps=reps)
                rec(key, t, 3 * a.nbytes, 8192, "reference", "full [8192x4096] LayerOps::add_forward")
            else:
                t = O.time_port(lambda: O.add(a, b), reps)
                rec(key, t, 3 * a.nbytes, 8192, "port", "full [8192x4096] oracle add")
        elif key == "cfg4_layernorm_bwd":
            x, g, b, eps = G.cfg4_layernorm(rows=512)
            dy = G.cfg4_grad((8192, 4096), 8)[:512]
            t = O.time_port(lambda: O.layernorm_bwd(x, dy, 4096, g, True, eps), reps)
            rec(key, t, 3 * x.nbytes + 5 * g.nbytes, 512, "port",
                "512 of 8192 rows, oracle layernorm_bwd (Model.cpp:7719-7821 restated)")
        elif key in ("cfg4_gelu_bwd", "cfg4_silu_bwd"):
            a = G.cfg4_gelu(rows=512)
            dy = G.cfg4_grad((8192, 11008), 9)[:512]
            fn = O.gelu_bwd if key == "cfg4_gelu_bwd" else O.silu_bwd
            t = O.time_port(lambda: fn(a, dy), reps)
            rec(key, t, 3 * a.nbytes, 512, "port", f"512 of 8192 rows, oracle {fn.__name__}")
        elif key == "cfg4_mul_bwd":
            g, u = G.cfg4_swiglu(rows=512)
            dy = G.cfg4_grad((8192, 11008), 10)[:512]
            t = O.time_port(lambda: O.mul_bwd(g, u, dy), reps)
            rec(key, t, 5 * g.nbytes, 512, "port", "512 of 8192 rows, oracle mul_bwd")
        elif key == "cfg4_add_bwd":
            a, _ = G.cfg4_add()
            t = O.time_port(lambda: (a.copy(), a.copy()), reps)
            rec(key, t, 3 * a.nbytes, 8192, "port",
                "full [8192x4096]: accumulate_grad into two absent names is two vector copies (Model.cpp:7552-7555)")
        elif key == "cfg3_safetensors_ingest":
            import struct
            import tempfile
            table, _ = G.cfg3_gather()
            hdr = json.dumps({"tok/weights": {"dtype": "F32", "shape": list(table.shape),
                                              "data_offsets": [0, table.nbytes]}}).encode()
            with tempfile.TemporaryDirectory() as d:
                path = os.path.join(d, "table.safetensors")
                with open(path, "wb") as f:
                    f.write(struct.pack("<Q", len(hdr)))
                    f.write(hdr)
                    f.write(table.tobytes())
                sys.path.insert(0, os.path.join(REPO, "oracle"))
                import model_ref as MR
                if MR.available():
                    layers = [dict(name="tok", type="Embedding", vocab_size=32000, embed_dim=4096,
                                   weights=np.zeros(table.size, np.float32))]
                    t = MR.time_safetensors_load(layers, path, reps)
                    rec(key, t, table.nbytes, 32000, "reference",
                        "Mimir::Serialization::load_checkpoint (SafeTensors, weights only) of the same file into "
                        "host weight blocks, page cache warm")
                else:
                    t = O.time_port(lambda: np.fromfile(path, np.uint8, count=table.nbytes, offset=8 + len(hdr)), reps)
                    rec(key, t, table.nbytes, 32000, "port", "sequential read of the tensor bytes into host memory")
        elif key in ("cfg4_runtime_block", "cfg4_runtime_block_fused"):
            rows = 1024
            x, res = G.cfg4_add(rows=rows)
            gate = G.cfg4_grad((8192, 4096), 11)[:rows]
            layers = block_layers()
            sys.path.insert(0, os.path.join(REPO, "oracle"))
            import model_ref as MR
            nb = 12 * x.nbytes + 2 * 4096 * 4
            if MR.available():
                t = MR.time_forward_named(layers, {"inp": x, "res": res, "gate": gate}, {}, reps)
                rec(key, t, nb, rows, "reference",
                    f"{rows} of 8192 rows: Model::forwardPassNamed of the same five layers (host tensor store)")
        elif key == "cfg4_runtime_block_train":
            rows = 256
            x, res = G.cfg4_add(rows=rows)
            gate = G.cfg4_grad((8192, 4096), 11)[:rows]
            lg = G.cfg4_grad((8192, 4096), 12)[:rows]
            sys.path.insert(0, os.path.join(REPO, "oracle"))
            import model_ref as MR
            if MR.available():
                t = MR.time_train_step(block_layers(), {"inp": x, "res": res, "gate": gate}, {}, lg, reps)
                rec(key, t, 31 * x.nbytes + 7 * 4096 * 4, rows, "reference",
                    f"{rows} of 8192 rows: Model::forwardPassNamed(training=true) then Model::backwardPass of the "
                    "same five layers (host tensor store)")
        elif key.endswith("_whole"):
            kind, x, w, eps, ref, port, _ = _whole_inputs(key)
            nb = 2 * x.nbytes + (w.nbytes if kind == "rmsnorm" else 0)
            if have_ref:
                rec(key, O.time_port(ref, reps), nb, 1, "reference",
                    f"the full 2^25-element row through the reference's {kind} layer function, median of {reps}")
            else:
                rec(key, O.time_port(port, reps), nb, 1, "port", f"the full 2^25-element row, oracle, median of {reps}")
        elif key == "f4_attention":
            # One (sequence, head) of the workload through the restatement of
            # the reference core (LayerOps.hpp:1045-1089, single-threaded as
            # the reference's core loops are); throughput in core flops.
            qkv = G.attention_qkv(1, 1024, 32, 128)
            q, k, v = (np.ascontiguousarray(qkv[:, i * 4096:i * 4096 + 128]) for i in range(3))
            t = O.time_port(lambda: O.attention(q, k, v, 1, True), reps)
            fl = attention_flops(1, 1, 1024, 1024, 128, True)
            out[key] = {"value": round(fl / t / 1e9, 3), "unit": "GFLOP/s", "seconds": round(t, 6),
                        "rows_per_s": round(1024 / t, 1), "cores": 1, "kind": "port",
                        "sample": "1 of 256 (sequence, head) pairs: 1024 causal queries, head_dim 128, "
                                  f"oracle_attention (bit-exact to the reference core), median of {reps}"}
        elif key == "f4_attention_bwd":
            # One (sequence, head) through the restatement of the reference's
            # backward core (Model.cpp:6892-7028, single-threaded as there).
            qkv = G.attention_qkv(1, 1024, 32, 128)
            q, k, v = (np.ascontiguousarray(qkv[:, i * 4096:i * 4096 + 128]) for i in range(3))
            do = np.ascontiguousarray(G.attention_dout(1, 1024, 32, 128)[:, :128])
            t = O.time_port(lambda: O.attention_bwd(q, k, v, do, 1, True), reps)
            fl = attention_bwd_flops(1, 1, 1024, 1024, 128, True)
            out[key] = {"value": round(fl / t / 1e9, 3), "unit": "GFLOP/s", "seconds": round(t, 6),
                        "rows_per_s": round(1024 / t, 1), "cores": 1, "kind": "port",
                        "sample": "1 of 256 (sequence, head) pairs: 1024 causal queries, head_dim 128, "
                                  f"oracle_attention_bwd (bit-exact to the reference's backward core), median of "
                                  f"{reps}"}
        elif key in ("cfg3_embedding_bwd", "cfg3_embedding_bwd_zipf"):
            ids = (G.cfg3_ids() if key == "cfg3_embedding_bwd" else G.cfg3_ids_zipf()).ravel()[:4096].copy()
            dy = G.cfg3_embedding_grad()[:4096].copy()
            gt = np.zeros(32000 * 4096, np.float32)
            fn = O._oracle().oracle_embedding_bwd_i32
            t = O.time_port(lambda: fn(O._p(ids), ids.size, O._p(dy), O._p(gt), gt.size, 32000, 4096, -1), reps)
            u = int(np.unique(ids).size)
            rec(key, t, ids.nbytes + dy.nbytes + 2 * u * 4096 * 4, 4096, "port",
                f"first 4096 of 32768 tokens ({u} distinct ids), oracle embedding_bwd_i32 into a resident table")
    return out


def _agreement(got, ref, bitexact, scale=None, exact=None):
    """Max |d| and max |d|/|ref| of got against ref, and whether every element
    meets the path's rule: NaN where ref is NaN, equal infinities, and
    |d| <= max(1e-6, 1e-5 |ref|) elsewhere (or equal bits, for the byte-exact
    ops).  For results that are float32 sums of many terms, `scale` is the sum
    of the terms' magnitudes and replaces |ref| where larger: two summation
    orders differ by ~u * scale however much the sum cancels.  With `exact`
    (the float64 value), an element outside the tolerance of ref also passes
    when it is within tolerance of exact and nearer to it than ref is: the
    reference's sequential float32 sums over very long rows carry errors of
    ~u*sqrt(n), beyond 1e-5 relative past ~10^4 terms."""
    g = np.ascontiguousarray(got, np.float32).ravel()
    r = np.ascontiguousarray(ref, np.float32).ravel()
    assert g.size == r.size, f"{g.size} != {r.size}"
    same_bits = bool(np.array_equal(g.view(np.uint32), r.view(np.uint32)))
    nan_ok = bool(np.array_equal(np.isnan(g), np.isnan(r)))
    inf_r = np.isinf(r)
    inf_ok = bool(np.array_equal(g[inf_r], r[inf_r]))
    fin = np.isfinite(r)
    g64, r64 = g[fin].astype(np.float64), r[fin].astype(np.float64)
    d = np.abs(g64 - r64)
    nz = r64 != 0
    mag = np.abs(r64) if scale is None else np.maximum(np.abs(r64), np.asarray(scale, np.float64).ravel()[fin])
    # An empty comparison proves nothing and does not pass.
    ok = d <= np.maximum(1e-6, 1e-5 * mag)
    if exact is not None:
        e64 = np.asarray(exact, np.float64).ravel()[fin]
        de = np.abs(g64 - e64)
        ok |= (de <= np.maximum(1e-6, 1e-5 * np.abs(e64))) & (de < np.abs(r64 - e64))
    within = bool(g.size > 0 and nan_ok and inf_ok and np.all(ok))
    same_bits = same_bits and g.size > 0
    rule = ("bit-identical" if bitexact else
            "|d| <= max(1e-6, 1e-5|ref|)" if scale is None else "|d| <= max(1e-6, 1e-5 max(|ref|, sum of |terms|))")
    if exact is not None:
        rule += ", or within that of the float64 value and nearer to it than ref"
    return {"elements": int(g.size), "max_abs": float(d.max()) if d.size else 0.0,
            "max_rel": float((d[nz] / np.abs(r64[nz])).max()) if nz.any() else 0.0,
            "bitexact": same_bits, "pass": same_bits if bitexact else within, "rule": rule}


def parity_leg(ctx, by_key, which):
    """Part of the cpu_baseline leg, as its checker: each op of `which` runs
    once more on freshly uploaded inputs through the same launch closure the
    timing used, and its output is compared with the CPU path's on the same
    inputs -- the reference's own functions (oracle/_ref) where the reference
    has one for the op, else the C restatement (oracle/lib).  Large configs
    compare the leading rows the CPU sample covers."""
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    import model_ref as MR
    have_ref = O.ref_available()
    out = {}

    def gpu_outputs(op, rows_like):
        step, sets = op.make(ctx, 1)
        try:
            step(0)
            ctx.sync()
            got = {}
            for name, dev in op.outputs(sets).items():
                like = rows_like[name]
                if isinstance(dev, np.ndarray):
                    got[name] = dev.ravel()[:like.size].reshape(like.shape)
                else:
                    host = np.empty(like.shape, dev.dtype)
                    ctx.download(host, dev)
                    got[name] = host
            return got
        finally:
            for bufs in sets:
                for b in bufs:
                    b.free()

    def check(key, refs, vs, sample, exact=(), scales=None, nearer=None):
        op = by_key[key]
        got = gpu_outputs(op, refs)
        scales = scales or {}
        nearer = nearer or {}
        res = {n: _agreement(got[n], refs[n], n in exact, scales.get(n), nearer.get(n)) for n in refs}
        out[key] = {"vs": vs, "sample": sample, "pass": all(r["pass"] for r in res.values()), "outputs": res}
        log(f"parity {key}: {'pass' if out[key]['pass'] else 'FAIL'} vs {vs} "
            + ", ".join(f"{n} max_abs {r['max_abs']:.3g}" for n, r in res.items()))

    def check_arrays(key, pairs, vs, sample):
        """pairs: {name: (got, ref, scale or None)} computed by the caller."""
        res = {n: _agreement(g, r, False, sc) for n, (g, r, sc) in pairs.items()}
        out[key] = {"vs": vs, "sample": sample, "pass": all(r["pass"] for r in res.values()), "outputs": res}
        log(f"parity {key}: {'pass' if out[key]['pass'] else 'FAIL'} vs {vs} "
            + ", ".join(f"{n} max_abs {r['max_abs']:.3g}" for n, r in res.items()))

    ref_or_port = "reference" if have_ref else "port"
    for key in which:
        if key not in by_key or (by_key[key].outputs is None and key != "cfg4_runtime_block_train"):
            continue
        if key in ("cfg0_layernorm", "cfg4_layernorm"):
            x, g, b, eps = G.cfg0_layernorm() if key == "cfg0_layernorm" else G.cfg4_layernorm(rows=1024)
            rows, cols = x.shape
            y = (O.ref_layernorm(x, cols, np.concatenate([g, b]), eps=eps) if have_ref
                 else O.layernorm(x, cols, g, b, eps))
            check(key, {"y": y.reshape(x.shape)}, ref_or_port, f"first {rows} rows")
        elif key == "cfg1_add_rmsnorm":
            x, r, w, eps = G.cfg1_add_rmsnorm()
            if have_ref:
                h = O.ref_add(x, r).reshape(x.shape)
                y = O.ref_rms_norm_rows(h, w, eps)
            else:
                y, h = O.add_rmsnorm(x, r, w, eps)
            check(key, {"y": y, "residual": h}, ref_or_port, "full [4096x4096]", exact=("residual",))
        elif key == "cfg2_softmax":
            s = G.cfg2_softmax(batch=1, heads=4).reshape(-1, 1024)
            y = O.ref_softmax_inplace(s) if have_ref else O.softmax_rows(s)
            check(key, {"y": y}, ref_or_port, "first 4096 of 262144 rows")
        elif key == "cfg3_gather":
            table, ids = G.cfg3_gather()
            ids = ids.ravel()[:4096].copy()
            if MR.available():
                # forwardPassNamed returns the tensor named "x"
                layers = [dict(name="tok", type="Embedding", inputs=["ids"], output="x", vocab_size=32000,
                               embed_dim=4096, weights=table.ravel())]
                y = MR.forward_named(layers, {}, {"ids": ids}, out_cap=ids.size * 4096)
                if y.size != ids.size * 4096:
                    raise RuntimeError(f"reference gather returned {y.size} floats, not {ids.size * 4096}")
                y = y.reshape(-1, 4096)
                vs = "reference (Model::forwardPassNamed, inline gather Model.cpp:1152-1205)"
            else:
                y, vs = O.embedding(ids, table, 32000, 4096, -1), "port"
            check(key, {"y": y}, vs, "first 4096 of 32768 tokens", exact=("y",))
        elif key == "cfg3_rope":
            q, k, theta = G.cfg3_rope(batch=1)
            c, s = O.rope_table(2048, 128, theta)
            check(key, {"q": O.rope(q, c, s), "k": O.rope(k, c, s)}, "port (no reference RoPE exists)",
                  "batch 1 of 16")
        elif key == "cfg4_gelu":
            a = G.cfg4_gelu(rows=512)
            y = O.ref_gelu(a) if have_ref else O.gelu(a)
            check(key, {"y": y.reshape(a.shape)}, ref_or_port, "first 512 of 8192 rows")
        elif key == "cfg4_silu_mul":
            g, u = G.cfg4_swiglu(rows=512)
            y = O.ref_mul(O.ref_silu(g), u) if have_ref else O.silu_mul(g, u)
            check(key, {"y": y.reshape(g.shape)}, ref_or_port, "first 512 of 8192 rows")
        elif key == "cfg4_add":
            a, b = G.cfg4_add()
            y = O.ref_add(a, b) if have_ref else O.add(a, b)
            check(key, {"y": y.reshape(a.shape)}, ref_or_port, "full [8192x4096]", exact=("y",))
        elif key == "cfg4_layernorm_bwd":
            x, g, b, eps = G.cfg4_layernorm()
            dy = G.cfg4_grad(x.shape, 8)
            dx, gp = O.layernorm_bwd(x, dy, 4096, g, True, eps)
            # Magnitudes of the terms each result sums (float64): dgamma and
            # dbeta add over 8192 rows; dx = inv/n (n dxh - sum dxh - xhat sum dxh xhat).
            x64, dy64 = x.astype(np.float64), dy.astype(np.float64)
            m = x64.mean(axis=1, keepdims=True)
            inv = 1.0 / np.sqrt(((x64 - m) ** 2).mean(axis=1, keepdims=True) + eps)
            xh = (x64 - m) * inv
            dxh = dy64 * g
            dx_scale = inv * (np.abs(dxh) + np.abs(dxh.mean(axis=1, keepdims=True))
                              + np.abs(xh * (dxh * xh).mean(axis=1, keepdims=True)))
            check(key, {"dx": dx.reshape(x.shape), "dgamma": gp[:4096], "dbeta": gp[4096:]}, "port",
                  "full [8192x4096]", scales={"dx": dx_scale, "dgamma": np.abs(dy64 * xh).sum(axis=0),
                                              "dbeta": np.abs(dy64).sum(axis=0)})
        elif key in ("cfg4_gelu_bwd", "cfg4_silu_bwd"):
            a = G.cfg4_gelu(rows=512)
            dy = G.cfg4_grad((8192, 11008), 9)[:512]
            fn = O.gelu_bwd if key == "cfg4_gelu_bwd" else O.silu_bwd
            check(key, {"dx": fn(a, dy)}, "port", "first 512 of 8192 rows")
        elif key == "cfg4_mul_bwd":
            g, u = G.cfg4_swiglu(rows=512)
            dy = G.cfg4_grad((8192, 11008), 10)[:512]
            da, db = O.mul_bwd(g, u, dy)
            check(key, {"da": da, "db": db}, "port", "first 512 of 8192 rows", exact=("da", "db"))
        elif key == "cfg4_add_bwd":
            a, _ = G.cfg4_add()
            check(key, {"da": a, "db": a}, "port (accumulate_grad into absent names copies dy)",
                  "full [8192x4096]", exact=("da", "db"))
        elif key.endswith("_whole"):
            # At 2^25 terms the reference's sequential float32 sums are
            # themselves off by up to a few percent, so the device is held to
            # the float64 value of the reference's formula and the
            # reference's own distance from it is reported beside.
            kind, x, _, _, ref, port, exact = _whole_inputs(key)
            shape = (8192, 4096)
            e = exact().reshape(shape)
            check(key, {"y": e}, "float64 value of the reference formula", "the full 2^25-element row")
            y = (ref() if have_ref else port()).reshape(shape)
            err = _agreement(y, e, False)
            out[key]["reference_error_vs_float64"] = {
                "of": ref_or_port, "max_abs": err["max_abs"], "max_rel": err["max_rel"]}
        elif key in ("cfg3_embedding_bwd", "cfg3_embedding_bwd_zipf"):
            # Ids with 32 tokens or more are summed in segments on the device:
            # their rows are float32 sums held to the sum-aware rule (scale:
            # the |dy| rows added), every other row bit for bit.
            ids = G.cfg3_ids() if key == "cfg3_embedding_bwd" else G.cfg3_ids_zipf()
            dy = G.cfg3_embedding_grad()
            z = np.zeros(32000 * 4096, np.float32)
            gt = O.embedding_bwd(ids, dy, z, 32000, 4096, -1)
            counts = np.bincount(ids.ravel(), minlength=32000)
            got = gpu_outputs(by_key[key], {"grad": gt})["grad"].reshape(32000, 4096)
            gt2 = gt.reshape(32000, 4096)
            short = counts < 32
            res = {"grad (ids < 32 tokens)": _agreement(got[short], gt2[short], True)}
            if (~short).any():
                sc = O.embedding_bwd(ids, np.abs(dy), z, 32000, 4096, -1).reshape(32000, 4096)
                res["grad (ids >= 32 tokens)"] = _agreement(got[~short], gt2[~short], False, sc[~short])
            out[key] = {"vs": "port", "sample": "full table [32000x4096], all 32768 tokens",
                        "pass": all(r["pass"] for r in res.values()), "outputs": res}
            log(f"parity {key}: {'pass' if out[key]['pass'] else 'FAIL'} vs port "
                + ", ".join(f"{n} max_abs {r['max_abs']:.3g}" for n, r in res.items()))
        elif key == "f4_attention":
            # Sampled (sequence, head) pairs of the full launch against the
            # restatement (pinned bit-exact to the reference core) with the
            # attention tolerance: 1e-5 of sum_j p_j |v_j| plus the propagated
            # rounding of the float32 scores, twice (both sides round).
            qkv = G.attention_qkv(8, 1024, 32, 128)
            got = gpu_outputs(by_key[key], {"out": np.empty((8192, 4096), np.float32)})["out"]
            res = {}
            for bi, h in ((0, 0), (3, 17), (7, 31)):
                rows = slice(bi * 1024, (bi + 1) * 1024)
                q, k, v = (np.ascontiguousarray(qkv[rows, i * 4096 + h * 128:i * 4096 + (h + 1) * 128])
                           for i in range(3))
                ref = O.attention(q, k, v, 1, True)
                _, mag, cond = O.attention_float64(q, k, v, 1, True, O.attention_scale(128))
                res[f"out (seq {bi}, head {h})"] = _agreement(got[rows, h * 128:(h + 1) * 128], ref, False,
                                                              mag + 2 * cond / 1e-5)
            res["out (first query of every head)"] = _agreement(
                got.reshape(8, 1024, 4096)[:, 0], qkv.reshape(8, 1024, 12288)[:, 0, 8192:], True)
            out[key] = {"vs": "port (oracle_attention, bit-exact to the reference's self_attention_forward core)",
                        "sample": "3 of 256 (sequence, head) pairs in full, and every head's first query "
                                  "(one visible key: V's row exactly)",
                        "pass": all(r["pass"] for r in res.values()), "outputs": res}
            log(f"parity {key}: {'pass' if out[key]['pass'] else 'FAIL'} vs port "
                + ", ".join(f"{n} max_abs {r['max_abs']:.3g}" for n, r in res.items()))
        elif key == "f4_attention_bwd":
            # Two (sequence, head) pairs of the full launch against the
            # restatement (bit-exact to the reference's backward core), each
            # element within twice the float64 model's first-order bound (both
            # sides round); every head's first query: dq is exactly 0 (one
            # visible key, so its dS row is 0).
            sys.path.insert(0, os.path.join(REPO, "tests"))
            from _attention import attention_bwd64
            qkv = G.attention_qkv(8, 1024, 32, 128)
            dout = G.attention_dout(8, 1024, 32, 128)
            got = gpu_outputs(by_key[key], {"dqkv": np.empty((8192, 12288), np.float32)})["dqkv"]
            res = {}
            for bi, h in ((0, 0), (7, 31)):
                rows = slice(bi * 1024, (bi + 1) * 1024)
                q, k, v = (np.ascontiguousarray(qkv[rows, i * 4096 + h * 128:i * 4096 + (h + 1) * 128])
                           for i in range(3))
                do = np.ascontiguousarray(dout[rows, h * 128:(h + 1) * 128])
                ref = O.attention_bwd(q, k, v, do, 1, True)
                _, tol = attention_bwd64(q, k, v, do, 1, True, O.attention_scale(128))
                for j, name in enumerate(("dq", "dk", "dv")):
                    cols = slice(j * 4096 + h * 128, j * 4096 + (h + 1) * 128)
                    res[f"{name} (seq {bi}, head {h})"] = _agreement(got[rows, cols], ref[j], False,
                                                                     2 * tol[j] / 1e-5)
            res["dq (first query of every sequence and head)"] = _agreement(
                got.reshape(8, 1024, 12288)[:, 0, :4096], np.zeros((8, 4096), np.float32), True)
            out[key] = {"vs": "port (oracle_attention_bwd, bit-exact to the reference's backward core)",
                        "sample": "2 of 256 (sequence, head) pairs in full (dq, dk, dv), and every head's "
                                  "first-query dq (exactly 0)",
                        "pass": all(r["pass"] for r in res.values()), "outputs": res}
            log(f"parity {key}: {'pass' if out[key]['pass'] else 'FAIL'} vs port "
                + ", ".join(f"{n} max_abs {r['max_abs']:.3g}" for n, r in res.items()))
        elif key == "cfg4_runtime_block_train" and MR.available():
            rows = 512
            x, res = G.cfg4_add(rows=rows)
            gate = G.cfg4_grad((8192, 4096), 11)[:rows]
            lg = G.cfg4_grad((8192, 4096), 12)[:rows]
            layers = block_layers()
            r_grads, _ = MR.backward(layers, {"inp": x, "res": res, "gate": gate}, {}, lg)
            ref = r_grads[1]  # the LayerNorm's [dgamma | dbeta]
            graph = M.DeviceGraph(ctx, layers)
            store = M.Store(ctx)
            dlg = ctx.to_device(lg)
            try:
                store.set_inputs({"inp": x, "res": res, "gate": gate}, {})
                store.run_training(graph)
                store.backward(graph, dlg)
                got = graph.grads()[1]
            finally:
                dlg.free()
                store.close()
                graph.close()
            # Magnitudes each float32 sum adds (float64 chain of the block):
            # dgamma = sum_rows dn*xhat, dbeta = sum_rows dn.
            g64, b64 = (np.asarray(layers[1]["weights"][:4096], np.float64),
                        np.asarray(layers[1]["weights"][4096:], np.float64))
            h = x.astype(np.float64) + res
            xh = (h - h.mean(axis=1, keepdims=True)) / np.sqrt(h.var(axis=1, keepdims=True) + 1e-5)
            n = xh * g64 + b64
            k = np.sqrt(np.float64(np.float32(2.0) / np.float32(3.14159265359)))
            t = np.tanh(k * (n + 0.044715 * n ** 3))
            gl = 0.5 * n * (1 + t)
            m = gl * gate
            s = 1 / (1 + np.exp(-m))
            dm = lg * (s + m * s * (1 - s))
            dn = dm * gate * (0.5 * (1 + t) + 0.5 * n * (1 - t * t) * k * (1 + 3 * 0.044715 * n * n))
            scale = np.concatenate([np.abs(dn * xh).sum(axis=0), np.abs(dn).sum(axis=0)])
            check_arrays(key, {"ln grad_weights": (got, ref, scale)},
                         "reference (Model::backwardPass of the same five layers)",
                         f"first {rows} of 8192 rows, the LayerNorm's [dgamma | dbeta] at the end of the chain")
        elif key in ("cfg4_runtime_block", "cfg4_runtime_block_fused") and MR.available():
            rows = 1024
            x, res = G.cfg4_add(rows=rows)
            gate = G.cfg4_grad((8192, 4096), 11)[:rows]
            layers = block_layers()
            y = MR.forward_named(layers, {"inp": x, "res": res, "gate": gate}, {})
            if y.size != x.size:
                raise RuntimeError(f"reference block returned {y.size} floats, not {x.size}")
            check(key, {"x": y}, "reference (Model::forwardPassNamed of the same five layers)",
                  f"first {rows} of 8192 rows")
    return out


def time_ingest(ctx, reps=3):
    """SafeTensors ingestion of the configs[3] embedding table (32000 x 4096
    fp32, 500 MiB) from a file straight into device memory
    (mimir_safetensors_read): the file is written to a temporary directory
    first, then read `reps` times (page cache warm after the first); the
    median read time gives GB/s.  Host-to-device bound (PCIe), not HBM."""
    import struct
    import tempfile
    import time
    table, _ = G.cfg3_gather()
    hdr = json.dumps({"tok/weights": {"dtype": "F32", "shape": list(table.shape),
                                      "data_offsets": [0, table.nbytes]}}).encode()
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "table.safetensors")
        with open(path, "wb") as f:
            f.write(struct.pack("<Q", len(hdr)))
            f.write(hdr)
            f.write(table.tobytes())
        dst = ctx.empty(table.shape)
        try:
            times = []
            with M.SafeTensors(ctx, path) as f:
                for _ in range(reps + 1):
                    t0 = time.perf_counter()
                    f.read("tok/weights", dst)
                    ctx.sync()
                    times.append(time.perf_counter() - t0)
            ok = bool(np.array_equal(dst.numpy()[:4], table[:4]))
        finally:
            dst.free()
    sec = float(np.median(times[1:]))
    return {"op": "cfg3_safetensors_ingest", "config": 3,
            "desc": "SafeTensors read of the embedding table [32000x4096] fp32 (500 MiB) file -> HBM",
            "kernel": "pinned double-buffered pread + hipMemcpyAsync", "algorithmic_bytes": int(table.nbytes),
            "us_per_launch": round(sec * 1e6, 1), "GB_s": round(table.nbytes / sec / 1e9, 2),
            "bound": "host-to-device (PCIe) and the page cache, not HBM", "first_read_s": round(times[0], 4),
            "reps": reps, "check": ok}


def load_traffic(workload):
    path = os.path.join(REPO, "profiles", f"traffic_{workload}.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="cfg1_add_rmsnorm")
    ap.add_argument("--op-steps", type=int, default=30, help="launches per op in the `ops` sweep")
    ap.add_argument("--ops", default="all", help="'all', 'none', or a comma list of op keys")
    ap.add_argument("--cpu", default="all", help="'all', 'workload' or 'none'")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--rows", type=int, default=None,
                    help="size sweeps only: rows of cfg1_add_rmsnorm / cfg4_layernorm (default: the configs')")
    ap.add_argument("--full-out", default=os.path.join("gpurun_out", "bench_full.json"),
                    help="file for the full per-op records ('' for none); stdout carries a summary")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one MI355X: this path has no multi-GPU form in this build "
              f"(--gpus {args.gpus}, WORLD_SIZE {world} requested); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    if args.rows is not None and args.cpu != "none":
        log("--rows is a size sweep: the CPU baseline and parity legs (configs' sizes) are skipped")
        args.cpu = "none"
    ops = build_ops(args.rows)
    by_key = {o.key: o for o in ops}
    if args.workload not in by_key:
        sys.exit(f"unknown workload {args.workload}; choose from {sorted(by_key)}")
    head = by_key[args.workload]
    if getattr(head, "bound", None) == "launch":
        sys.exit(f"{args.workload} is launch-bound (it is timed in the sweep, not as the metric's workload)")

    ctx = M.Context(0)
    log(f"workload {head.key}: {head.desc}")
    res = time_op(ctx, head, args.steps, args.warmup)
    log(f"  {res['us_per_launch']} us/launch, {res['GB_s']} GB/s ({100 * res['frac_of_peak']:.1f}% of peak)")

    # The practical ceiling at this size: a plain copy moving the same bytes
    # per launch (half read, half written), timed the same way.
    copies = {}
    same = same_bytes_copy(ctx, head.nbytes, args.steps, args.warmup, copies)
    log(f"  copy of the same bytes: {same['us_per_launch']} us/launch, {same['GB_s']} GB/s")

    sweep = []
    keys = ([o.key for o in ops] if args.ops == "all" else
            [] if args.ops == "none" else args.ops.split(","))
    for k in keys:
        if k == head.key:
            res["copy_same_bytes_GB_s"] = same["GB_s"]
            res["frac_of_copy"] = round(res["GB_s"] / same["GB_s"], 4)
            sweep.append(res)
            continue
        if k == "cfg3_safetensors_ingest":
            continue
        r = time_op(ctx, by_key[k], args.op_steps, 3)
        if k in QUEUED_OPS:
            q = time_queued(ctx, by_key[k])
            r.update({"host_driven": {"us_per_launch": r["us_per_launch"], "GB_s": r["GB_s"],
                                      "note": "host-bound: one Python call per launch"},
                      "us_per_launch": q["us_per_launch"], "GB_s": q["GB_s"],
                      "frac_of_peak": q["frac_of_peak"], "timing": q["method"],
                      "rows_per_s": round(by_key[k].rows / (q["us_per_launch"] * 1e-6), 1)})
            log(f"op {k}: {r['us_per_launch']} us/launch on the GPU ({100 * r['frac_of_peak']:.1f}%); "
                f"{r['host_driven']['us_per_launch']} us/launch host-driven (host-bound)")
        elif r.get("bound") == "launch":
            log(f"op {k}: {r['us_per_launch']} us/launch (launch-bound)")
        else:
            log(f"op {k}: {r['us_per_launch']} us/launch, {r['GB_s']} GB/s ({100 * r['frac_of_peak']:.1f}%)")
        if r.get("bound") not in ("mfma", "launch") and k not in QUEUED_OPS and k != "calib_copy":
            c = same_bytes_copy(ctx, by_key[k].nbytes, args.op_steps, 3, copies)
            r["copy_same_bytes_GB_s"] = c["GB_s"]
            r["frac_of_copy"] = round(r["GB_s"] / c["GB_s"], 4)
        sweep.append(r)
    if args.ops == "all" or "cfg3_safetensors_ingest" in keys:
        r = time_ingest(ctx)
        log(f"op cfg3_safetensors_ingest: {r['us_per_launch']} us, {r['GB_s']} GB/s (first read {r['first_read_s']} s)")
        sweep.append(r)
        if "cfg3_safetensors_ingest" not in keys:
            keys = keys + ["cfg3_safetensors_ingest"]

    cpu, parity = {}, {}
    if args.cpu != "none":
        which = [head.key] if args.cpu == "workload" else keys or [head.key]
        try:
            cpu = cpu_leg(which, args.cpu_reps)
        except Exception as e:  # the baseline is reported, never required
            log(f"cpu baseline unavailable: {e}")
        try:
            parity = parity_leg(ctx, by_key, which)
        except Exception as e:
            log(f"parity check unavailable: {e}")
    ctx.close()
    for r in sweep:
        if r["op"] in cpu:
            c = cpu[r["op"]]
            r["cpu_kind"] = c["kind"]
            r["cpu_us_sample"] = round(c["seconds"] * 1e6, 1)
            r["cpu_sample"] = c["sample"]
            if c["unit"] == "GFLOP/s":
                r["cpu_GFLOP_s"] = c["value"]
                r["speedup_vs_cpu"] = round(r["TFLOP_s"] * 1e3 / c["value"], 1)
            else:
                r["cpu_GB_s"] = c["value"]
                r["speedup_vs_cpu"] = round(r["GB_s"] / c["value"], 1)
        if r["op"] in parity:
            r["parity"] = parity[r["op"]]

    for r in sweep:
        t = load_traffic(r["op"])
        if t is not None:
            r["traffic_bytes"] = t["traffic_bytes"]
            r["traffic_over_algorithmic"] = t["traffic_over_algorithmic"]
            if "distinct_row_bytes" in t:
                # The gather counted by the table rows it must read at least
                # once (repeated ids may be served by L2 or the Infinity Cache).
                r["distinct_row_bytes"] = t["distinct_row_bytes"]
                r["distinct_row_GB_s"] = round(t["distinct_row_bytes"] / (r["us_per_launch"] * 1e3), 1)
                r["distinct_row_frac_of_peak"] = round(r["distinct_row_GB_s"] / PEAK_GBS, 4)

    traffic = load_traffic(head.key)
    host = {"cpu_model": cpu_model(), "nproc": os.cpu_count()}
    cb = cpu.get(head.key)
    line = {
        "metric": METRIC,
        "value": res["GB_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(res["us_per_launch"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,1) inputs of the BASELINE configs (numpy PCG64), resident in HBM",
        "config": {
            "workload": (f"configs[{head.config}]: {head.desc}" if head.config >= 0 else head.desc),
            "op": head.key,
            "algorithmic_bytes_per_step": head.nbytes,
            "rows_per_step": head.rows,
            "buffer_sets": res["buffer_sets"],
            "footprint_MiB": res["footprint_MiB"],
            "mall": "buffer sets rotated so one pass exceeds 1.25 GiB (Infinity Cache 256 MiB)",
            "clock_spin_up_s": 0.25,
        },
        "rows_per_s": res["rows_per_s"],
        "frac_of_peak": res["frac_of_peak"],
        "roofline": ({
            "bound": "mfma",
            "kernel": head.kernel,
            "achieved": res["TFLOP_s"],
            "peak": PEAK_F32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": res["frac_of_peak"],
            "traffic": None if traffic is None else traffic.get("traffic_bytes"),
            "algorithmic_flops": head.flops,
            "algorithmic_bytes": head.nbytes,
        } if head.flops else {
            "bound": "hbm",
            "kernel": head.kernel,
            "achieved": res["GB_s"],
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": res["frac_of_peak"],
            "traffic": None if traffic is None else traffic.get("traffic_bytes"),
            "algorithmic_bytes": head.nbytes,
            "copy_same_bytes": {"GB_s": same["GB_s"], "frac": same["frac_of_peak"],
                                "us_per_launch": same["us_per_launch"]},
            "frac_of_copy": round(res["GB_s"] / same["GB_s"], 4),
        }),
        "cpu_baseline": None if cb is None else {
            "value": cb["value"], "unit": cb["unit"], "cores": cb["cores"], "kind": cb["kind"],
            "sample": cb["sample"], "rows_per_s": cb["rows_per_s"], **host},
        "parity": compact_parity(parity.get(head.key)),
        "ops_fields": ["us_per_launch", "GB_s", "frac_of_peak", "parity_pass", "traffic_over_algorithmic",
                       "frac_of_copy"],
        "ops": {r["op"]: [r["us_per_launch"], r["GB_s"], r.get("frac_of_peak"),
                          r["parity"]["pass"] if "parity" in r else None,
                          r.get("traffic_over_algorithmic"), r.get("frac_of_copy")]
                for r in sweep if r.get("bound") not in ("mfma", "launch")},
        "mfma_ops_fields": ["us_per_launch", "TFLOP_s", "frac_of_fp32_mfma_peak", "parity_pass",
                            "cpu_GFLOP_s"],
        "mfma_ops": {r["op"]: [r["us_per_launch"], r["TFLOP_s"], r["frac_of_peak"],
                               r["parity"]["pass"] if "parity" in r else None, r.get("cpu_GFLOP_s")]
                     for r in sweep if r.get("bound") == "mfma"},
    }
    stack = {r["op"]: r["us_per_launch"] for r in sweep if r.get("bound") == "launch"}
    if "f1_stack_eager" in stack and "f1_stack_graph" in stack:
        line["runtime_graph"] = {"layers": 20, "eager_us": stack["f1_stack_eager"],
                                 "graph_us": stack["f1_stack_graph"],
                                 "speedup": round(stack["f1_stack_eager"] / stack["f1_stack_graph"], 2)}
    full = dict(line, parity=parity.get(head.key), ops=sweep)
    out = args.full_out
    if out:
        os.makedirs(os.path.dirname(os.path.abspath(out)), exist_ok=True)
        with open(out, "w") as f:
            json.dump(full, f, indent=1)
        line["full_records"] = os.path.relpath(os.path.abspath(out), REPO)
        log(f"full per-op records written to {out}")
    text = json.dumps(line, separators=(",", ":"))
    if len(text) > STDOUT_LIMIT:
        # The driver keeps the tail of stdout; a line it cannot parse whole
        # loses the measurement.  The per-op summary goes first.
        line.pop("ops")
        text = json.dumps(line, separators=(",", ":"))
    print(text, flush=True)


def compact_parity(p):
    """The headline's parity record without the per-output rule strings."""
    if p is None:
        return None
    return {"vs": p["vs"], "sample": p["sample"], "pass": p["pass"],
            "outputs": {n: {k: o[k] for k in ("max_abs", "max_rel", "bitexact", "pass")}
                        for n, o in p["outputs"].items()}}


if __name__ == "__main__":
    main()
