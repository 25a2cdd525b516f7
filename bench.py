"""Benchmark of the sparse-voxel convolution path on one MI355X.

Default workload (the north-star target): 2x sparse
subdivide of ~0.32M R=256 shell parents (Bernoulli(0.5) per child) into ~1.26M
R=512 children, hash + kernel map of the children, parent->child feature
broadcast (skip_repeat 256->256) and a 3x3x3 submanifold conv 256->128, all in
bf16 storage with fp32 accumulation.  One step = that whole chain, with every
input (parent coordinates, logits, parent features, weights) resident in HBM
when the timed region starts.

Prints one JSON line.  `value` is whole-step effective conv TFLOP/s
(2*P*Ci*Co per step / step time); `roofline` is the conv kernel's own rate from
HIP events recorded on the backend stream around each conv launch;
`cpu_baseline` is the single-threaded CPU oracle (a restatement of the
reference CPU backend) on a bounded sample of the same workload.
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "trellis2.c_amd"))

import numpy as np  # noqa: E402

import sparse_hip as sh  # noqa: E402
import workloads as wl  # noqa: E402

PEAK_TFLOPS = {sh.F32: 157.3, sh.F16: 2516.6, sh.BF16: 2516.6}
PEAK_HBM_GBS = 8000.0
METRIC = "submanifold conv effective TFLOP/s + hash/kernel-map Mvoxels/s, 1 MI355X"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Cfg3:
    """Subdivide -> hash/map -> broadcast -> conv on device-resident inputs."""

    def __init__(self, be, w):
        self.be = be
        self.w = w
        dt = be.dtype
        self.parents = w["parent_coords"].shape[0]
        self.pmap = be.upload_coords(w["parent_coords"])
        self.logits = be.upload(w["logits"])
        self.pfeats = be.upload(w["parent_feats"])
        self.weight = be.keep(np.ascontiguousarray(w["weight"], np.float32))
        self.ci, self.co = w["ci"], w["co"]
        # Size the child buffers once from a first pass (not timed).
        dm = be.build_c2s_map_device(self.logits, self.parents, coords_map=self.pmap)
        self.m = dm.n
        rb = be.build_rulebook_for_c2s_map(dm)
        self.pairs = be.rulebook_stats(rb)["pairs"]
        rb.free()
        be.free_map(dm)
        self.xc = be.alloc(self.m * self.ci)
        self.y = be.alloc(self.m * self.co)
        self.dtype = dt

    def step(self):
        be = self.be
        dm = be.build_c2s_map_device(self.logits, self.parents, coords_map=self.pmap)
        rb = be.build_rulebook_for_c2s_map(dm)
        be.skip_repeat_device(self.pfeats, dm, self.xc, self.ci, self.ci)
        be.conv(rb, self.xc, self.weight, None, self.y, self.ci, self.co)
        rb.free()
        be.free_map(dm)

    def describe(self):
        return {"workload": self.w["name"], "parents": int(self.parents), "voxels": int(self.m),
                "pairs": int(self.pairs), "ci": self.ci, "co": self.co, "grid": "R=256 -> R=512",
                "subdivide": "Bernoulli(0.5) per child", "broadcast": "skip_repeat 256->256"}

    def flops(self):
        return wl.conv_flops(self.pairs, self.ci, self.co)


class ConvOnly:
    """Configs 1, 4, 5: hash + kernel map rebuild and one conv per step."""

    def __init__(self, be, w):
        self.be = be
        self.w = w
        self.n = w["coords"].shape[0]
        self.cmap = be.upload_coords(w["coords"])
        self.x = be.upload(w["feats"])
        self.weight = be.keep(np.ascontiguousarray(w["weight"], np.float32))
        self.ci, self.co = w["ci"], w["co"]
        self.y = be.alloc(self.n * self.co)
        rb = be.build_rulebook_for_c2s_map(self.cmap)
        self.pairs = be.rulebook_stats(rb)["pairs"]
        rb.free()
        self.m = self.n

    def step(self):
        rb = self.be.build_rulebook_for_c2s_map(self.cmap)
        self.be.conv(rb, self.x, self.weight, None, self.y, self.ci, self.co)
        rb.free()

    def describe(self):
        return {"workload": self.w["name"], "voxels": int(self.n), "pairs": int(self.pairs), "ci": self.ci,
                "co": self.co}

    def flops(self):
        return wl.conv_flops(self.pairs, self.ci, self.co)


class Cfg2(ConvOnly):
    """Residual block: conv -> LayerNorm -> SiLU -> conv -> + skip (fp16).

    By default the two slot pairs run as the fused entry points
    trellis_sparse_hip_conv_norm and trellis_sparse_hip_conv_add (the norm and
    the add happen in the convs' epilogues); --slots runs the four slots."""

    def __init__(self, be, w, slots=False):
        super().__init__(be, w)
        self.slots = slots
        self.weight2 = be.keep(np.ascontiguousarray(w["weight2"], np.float32))
        self.gamma = be.keep(w["gamma"])
        self.beta = be.keep(w["beta"])
        self.h = be.alloc(self.n * self.co)
        self.out = be.alloc(self.n * self.co)

    def step(self):
        be = self.be
        rb = be.build_rulebook_for_c2s_map(self.cmap)
        if self.slots:
            be.conv(rb, self.x, self.weight, None, self.y, self.ci, self.co)
            be.row_norm(self.y, self.gamma, self.beta, self.h, self.n, self.co, 1e-6, silu=True)
            be.conv(rb, self.h, self.weight2, None, self.y, self.co, self.co)
            be.add(self.y, self.x, self.out, self.n * self.co)
        else:
            be.conv_norm(rb, self.x, self.weight, None, self.gamma, self.beta, 1e-6, self.h, self.ci, self.co,
                         silu=True)
            be.conv_add(rb, self.h, self.weight2, None, self.x, self.out, self.co, self.co)
        rb.free()

    def describe(self):
        d = super().describe()
        d["block"] = ("conv -> row_norm_silu -> conv -> add (slots)" if self.slots else
                      "conv_norm(silu) -> conv_add (fused epilogues)")
        return d

    def flops(self):
        return 2 * wl.conv_flops(self.pairs, self.ci, self.co)


class Block:
    """Decoder blocks composed from the backend's slots, at config-3 scale (bf16).

    convnext: on the ~1.26M config-3 children, C = 128:
      conv(128->128) -> row_norm -> linear_silu(128->512) -> linear(512->128) -> add
      (src/architectures/sparse_unet_decoder/executor.c:176-255).  With
      --channels 256: on the ~0.32M config-3 parents, C = 256 (the decoder
      level above the children, decoder.c:248-249); --channels 512: on the
      parents' own parents (the parent coordinates halved, ~0.08M voxels),
      C = 512, the level above that, whose tail runs composed (row_norm and
      the two linears through the GEMM library, the residual in the second
      one's epilogue).
    convnext_fused: the same block with its tail (row_norm .. add) in the one
      fused entry point trellis_sparse_hip_convnext_mlp.
    convnext_block: the whole block in one call, trellis_sparse_hip_convnext_block
      (the conv into one intermediate, then the fused tail).
    s2c: the encoder's S2C down-block on the ~1.26M config-3 children, Ci = 64 -> Co = 128
      (sparse_unet_encoder/executor.c:160-360): row_norm_silu -> conv(64->16) on the fine
      rulebook; S2C map, pack and skip mean on the device (the reference does these on
      the host, s2c_host.c:33-120, executor.c:258-300); coarse rulebook; row_norm_silu
      -> conv(128->128) on the coarse voxels -> add(skip).  The line also carries the
      CPU oracle's S2C map time on the same voxels.
    mesh: FlexiDualGrid mesh extraction (src/ops/mesh/flex_dual_grid.c:166-313) from
      7-channel decoder logits on the ~1.26M config-3 children (R = 512), coordinates
      and logits resident on the device, vertices and faces returned as host arrays
      (the reference function's contract); the CPU oracle beside it.
    c2s: the C2S up-block on the ~0.32M config-3 parents, Ci = 256 -> Co = 128:
      linear(256->8) logits -> build_c2s_map_device -> build_rulebook_for_c2s_map;
      row_norm_silu -> conv(256->1024) on the parents -> c2s_gather_device;
      skip_repeat_device; row_norm_silu -> conv(128->128) on the children -> add
      (executor.c:257-554).
    In c2s and s2c the closing conv -> add runs as one trellis_sparse_hip_conv_add
    (slot "conv_add_post") unless --slots is given.
    Slot times come from HIP events on the backend stream between slots (every
    slot runs on that stream, in call order).
    """

    def __init__(self, be, kind, slots=False, channels=128):
        self.be, self.kind, self.fuse_add = be, kind, not slots
        w = wl.workload(3)
        rng = np.random.default_rng(11)
        f32 = lambda a: np.ascontiguousarray(a, np.float32)
        if kind in ("convnext", "convnext_fused", "convnext_block"):
            c = channels
            if c == 512:
                pc = w["parent_coords"].copy()
                pc[:, 1:] >>= 1
                pmap = be.upload_coords(np.ascontiguousarray(np.unique(pc, axis=0), dtype=np.int32))
            else:
                pmap = be.upload_coords(w["parent_coords"])
            if c == 128:
                dm = be.build_c2s_map_device(be.upload(w["logits"]), w["parent_coords"].shape[0], coords_map=pmap)
            else:
                dm = pmap
            self.cmap, self.n, self.c = dm, dm.n, c
            self.h = be.upload(rng.standard_normal((self.n, c)).astype(np.float32))
            self.conv_w = be.keep(f32(rng.standard_normal((c, 27, c)) / np.sqrt(27 * c)))
            self.conv_b = be.keep(f32(0.1 * rng.standard_normal(c)))
            self.gamma = be.keep(f32(1 + 0.1 * rng.standard_normal(c)))
            self.beta = be.keep(f32(0.1 * rng.standard_normal(c)))
            self.w0 = be.keep(f32(rng.standard_normal((4 * c, c)) / np.sqrt(c)))
            self.b0 = be.keep(f32(0.1 * rng.standard_normal(4 * c)))
            self.w2 = be.keep(f32(rng.standard_normal((c, 4 * c)) / np.sqrt(4 * c)))
            self.b2 = be.keep(f32(0.1 * rng.standard_normal(c)))
            self.rb = be.build_rulebook_for_c2s_map(self.cmap)
            self.pairs = be.rulebook_stats(self.rb)["pairs"]
            self.bufs = [be.alloc(self.n * c), be.alloc(self.n * c), be.alloc(self.n * 4 * c),
                         be.alloc(self.n * c), be.alloc(self.n * c)]
            self.slots = ["sparse_conv3d", "row_norm", "linear_silu", "linear", "add"]
            if kind == "convnext_fused":
                self.slots = ["sparse_conv3d", "convnext_mlp"]
            if kind == "convnext_block":
                self.slots = ["convnext_block"]
        elif kind == "mesh":
            pmap = be.upload_coords(w["parent_coords"])
            dm = be.build_c2s_map_device(be.upload(w["logits"]), w["parent_coords"].shape[0], coords_map=pmap)
            self.cmap, self.n = dm, dm.n
            self.coords = be.download_c2s_coords(dm)
            self.logits7 = rng.standard_normal((self.n, 7)).astype(np.float32) * 2
            self.feats = be.upload(self.logits7)
            self.faces = 0
            self.slots = ["flex_dual_grid_mesh"]
        elif kind == "s2c":
            ci, co = 64, 128
            self.ci, self.co = ci, co
            pmap = be.upload_coords(w["parent_coords"])
            dm = be.build_c2s_map_device(be.upload(w["logits"]), w["parent_coords"].shape[0], coords_map=pmap)
            self.fine_map, self.n = dm, dm.n
            self.frb = be.build_rulebook_for_c2s_map(dm)
            self.fpairs = be.rulebook_stats(self.frb)["pairs"]
            self.h = be.upload(rng.standard_normal((self.n, ci)).astype(np.float32))
            self.g1 = be.keep(f32(1 + 0.1 * rng.standard_normal(ci)))
            self.b1 = be.keep(f32(0.1 * rng.standard_normal(ci)))
            self.w1 = be.keep(f32(rng.standard_normal((co // 8, 27, ci)) / np.sqrt(27 * ci)))
            self.c1b = be.keep(f32(0.1 * rng.standard_normal(co // 8)))
            self.w2 = be.keep(f32(rng.standard_normal((co, 27, co)) / np.sqrt(27 * co)))
            self.c2b = be.keep(f32(0.1 * rng.standard_normal(co)))
            self.norm1 = be.alloc(self.n * ci)
            self.conv1 = be.alloc(self.n * (co // 8))
            fmap, cmap = be.s2c_build_device(coords_map=dm)
            self.m = cmap.n
            crb = be.build_rulebook_for_c2s_map(cmap)
            self.pairs = be.rulebook_stats(crb)["pairs"]
            crb.free()
            self.fine_coords = be.download_c2s_coords(dm)
            be.free_map(fmap)
            be.free_map(cmap)
            self.bufs = [be.alloc(self.m * co) for _ in range(5)]
            self.slots = ["row_norm_silu_pre", "sparse_conv3d_pre", "s2c_build_device", "s2c_pack_device",
                          "s2c_skip_mean_device", "build_rulebook_for_c2s_map", "row_norm_silu_post",
                          "sparse_conv3d_post", "add"]
            if self.fuse_add:
                self.slots[-2:] = ["conv_add_post"]
        else:
            ci, co = 256, 128
            self.ci, self.co = ci, co
            self.n = w["parent_coords"].shape[0]
            self.pmap = be.upload_coords(w["parent_coords"])
            self.prb = be.build_rulebook_for_c2s_map(self.pmap)
            self.ppairs = be.rulebook_stats(self.prb)["pairs"]
            self.h = be.upload(w["parent_feats"])
            self.ws = be.keep(f32(rng.standard_normal((8, ci)) / np.sqrt(ci)))
            self.bs = be.keep(f32(0.1 * rng.standard_normal(8)))
            self.g1 = be.keep(f32(1 + 0.1 * rng.standard_normal(ci)))
            self.b1 = be.keep(f32(0.1 * rng.standard_normal(ci)))
            self.w1 = be.keep(f32(rng.standard_normal((8 * co, 27, ci)) / np.sqrt(27 * ci)))
            self.c1b = be.keep(f32(0.1 * rng.standard_normal(8 * co)))
            self.w2 = be.keep(f32(rng.standard_normal((co, 27, co)) / np.sqrt(27 * co)))
            self.c2b = be.keep(f32(0.1 * rng.standard_normal(co)))
            self.subdiv = be.alloc(self.n * 8)
            self.norm1 = be.alloc(self.n * ci)
            self.conv1 = be.alloc(self.n * 8 * co)
            be.linear(self.h, self.ws, self.bs, self.subdiv, self.n, ci, 8)
            dm = be.build_c2s_map_device(self.subdiv, self.n, coords_map=self.pmap)
            self.m = dm.n
            rb = be.build_rulebook_for_c2s_map(dm)
            self.pairs = be.rulebook_stats(rb)["pairs"]
            rb.free()
            be.free_map(dm)
            self.bufs = [be.alloc(self.m * co) for _ in range(5)]
            self.slots = ["linear_subdiv", "build_c2s_map_device", "build_rulebook_for_c2s_map", "row_norm_silu_pre",
                          "sparse_conv3d_pre", "c2s_gather_device", "skip_repeat_device", "row_norm_silu_post",
                          "sparse_conv3d_post", "add"]
            if self.fuse_add:
                self.slots[-2:] = ["conv_add_post"]

    def step(self):
        be = self.be
        ev = iter(range(1, 16))
        be.event(0)
        if self.kind == "mesh":
            _, f = be.flex_dual_grid_mesh(self.feats, self.n, 7, 512, coords_map=self.cmap)
            self.faces = f.shape[0]
            be.event(next(ev))
            return
        if self.kind == "s2c":
            n, ci, co, m = self.n, self.ci, self.co, self.m
            packed, skip, norm2, conv2, out = self.bufs
            be.row_norm(self.h, self.g1, self.b1, self.norm1, n, ci, 1e-6, silu=True)
            be.event(next(ev))
            be.conv(self.frb, self.norm1, self.w1, self.c1b, self.conv1, ci, co // 8)
            be.event(next(ev))
            fmap, cmap = be.s2c_build_device(coords_map=self.fine_map)
            be.event(next(ev))
            be.s2c_pack_device(self.conv1, fmap, packed, co)
            be.event(next(ev))
            be.s2c_skip_mean_device(self.h, fmap, skip, ci, co)
            be.event(next(ev))
            rb = be.build_rulebook_for_c2s_map(cmap)
            be.event(next(ev))
            be.row_norm(packed, None, None, norm2, m, co, 1e-6, silu=True)
            be.event(next(ev))
            if self.fuse_add:
                be.conv_add(rb, norm2, self.w2, self.c2b, skip, out, co, co)
                be.event(next(ev))
            else:
                be.conv(rb, norm2, self.w2, self.c2b, conv2, co, co)
                be.event(next(ev))
                be.add(conv2, skip, out, m * co)
                be.event(next(ev))
            rb.free()
            be.free_map(fmap)
            be.free_map(cmap)
            return
        if self.kind == "convnext_block":
            be.convnext_block(self.rb, self.h, self.conv_w, self.conv_b, self.gamma, self.beta, self.w0, self.b0,
                              self.w2, self.b2, self.bufs[4], self.c, 1e-6)
            be.event(next(ev))
            return
        if self.kind == "convnext_fused":
            conv, out = self.bufs[0], self.bufs[4]
            be.conv(self.rb, self.h, self.conv_w, self.conv_b, conv, self.c, self.c)
            be.event(next(ev))
            be.convnext_mlp(conv, self.gamma, self.beta, self.w0, self.b0, self.w2, self.b2, self.h, out, self.n,
                            self.c, 1e-6)
            be.event(next(ev))
            return
        if self.kind == "convnext":
            n, c = self.n, self.c
            conv, norm, mlp1, mlp2, out = self.bufs
            be.conv(self.rb, self.h, self.conv_w, self.conv_b, conv, c, c)
            be.event(next(ev))
            be.row_norm(conv, self.gamma, self.beta, norm, n, c, 1e-6)
            be.event(next(ev))
            be.linear(norm, self.w0, self.b0, mlp1, n, c, 4 * c, silu=True)
            be.event(next(ev))
            be.linear(mlp1, self.w2, self.b2, mlp2, n, 4 * c, c)
            be.event(next(ev))
            be.add(self.h, mlp2, out, n * c)
            be.event(next(ev))
            return
        n, ci, co = self.n, self.ci, self.co
        be.linear(self.h, self.ws, self.bs, self.subdiv, n, ci, 8)
        be.event(next(ev))
        dm = be.build_c2s_map_device(self.subdiv, n, coords_map=self.pmap)
        be.event(next(ev))
        rb = be.build_rulebook_for_c2s_map(dm)
        be.event(next(ev))
        be.row_norm(self.h, self.g1, self.b1, self.norm1, n, ci, 1e-6, silu=True)
        be.event(next(ev))
        be.conv(self.prb, self.norm1, self.w1, self.c1b, self.conv1, ci, 8 * co)
        be.event(next(ev))
        h_up, skip, norm2, conv2, out = self.bufs
        be.c2s_gather_device(self.conv1, dm, h_up, co)
        be.event(next(ev))
        be.skip_repeat_device(self.h, dm, skip, ci, co)
        be.event(next(ev))
        be.row_norm(h_up, None, None, norm2, self.m, co, 1e-6, silu=True)
        be.event(next(ev))
        if self.fuse_add:
            be.conv_add(rb, norm2, self.w2, self.c2b, skip, out, co, co)
            be.event(next(ev))
        else:
            be.conv(rb, norm2, self.w2, self.c2b, conv2, co, co)
            be.event(next(ev))
            be.add(conv2, skip, out, self.m * co)
            be.event(next(ev))
        rb.free()
        be.free_map(dm)

    def flops(self):
        if self.kind == "mesh":
            return 0
        if self.kind == "s2c":
            return wl.conv_flops(self.fpairs, self.ci, self.co // 8) + wl.conv_flops(self.pairs, self.co, self.co)
        if self.kind in ("convnext", "convnext_fused", "convnext_block"):
            n, c = self.n, self.c
            return wl.conv_flops(self.pairs, c, c) + 2 * (2 * n * c * 4 * c)
        return (wl.conv_flops(self.ppairs, self.ci, 8 * self.co) + wl.conv_flops(self.pairs, self.co, self.co)
                + 2 * self.n * self.ci * 8)


def random_weights(be, rng):
    """Two makers of device-cached random fp32 weights: rnd(shape, fan_in) ~ N(0, 1/fan_in); small(count) ~ N(0,
    0.1), or 1 + N(0, 0.1) with one=True (norm scales)."""

    def rnd(shape, fan_in):
        return be.keep(np.ascontiguousarray(rng.standard_normal(shape, dtype=np.float32) / np.float32(np.sqrt(fan_in))))

    def small(count, scale=0.1, one=False):
        v = rng.standard_normal(count, dtype=np.float32) * np.float32(scale)
        return be.keep(np.ascontiguousarray(v + np.float32(1) if one else v))

    return rnd, small


class Decoder:
    """The whole shape decoder of the sparse U-Net VAE at the reference's widths, through the backend's entry
    points in the executor's order (src/architectures/sparse_unet_decoder/decoder.c:248-249: channels
    {1024, 512, 256, 128, 64}, ConvNeXt blocks {4, 16, 8, 4, 0}; executor.c:560-760):
      from_latent linear 32 -> 1024 and the rulebook on the latent voxels;
      per level its ConvNeXt blocks (trellis_sparse_hip_convnext_block: fused tail at 256 and below, composed
      at 512 and 1024), then a C2S up-block to the next width (subdivision logits linear(Ci -> 8) ->
      build_c2s_map_device -> build_rulebook_for_c2s_map; row_norm_silu -> conv(Ci -> 8 Co) on the parents ->
      c2s_gather_device; skip_repeat_device; row_norm_silu -> conv(Co -> Co) + the skip, as one
      trellis_sparse_hip_conv_add where Co % 128 == 0, else conv and add);
      the output head: row_norm (eps 1e-5, no affine) -> linear 64 -> 7.
    Latent voxels: the config-3 parent shell (R = 256) reduced to R = 64 (coordinates >> 2, unique), 32 random
    channels.  Every layer has its own random weights; the subdivision logits come from random weights with
    zero bias, so each up-block keeps about half of the children (about four times the parent count).
    """

    CHANNELS = (1024, 512, 256, 128, 64)
    BLOCKS = (4, 16, 8, 4, 0)
    LATENT = 32
    OUT = 7

    def __init__(self, be):
        self.be = be
        rng = np.random.default_rng(17)
        w = wl.workload(3)
        pc = w["parent_coords"].copy()
        pc[:, 1:] >>= 2
        self.coords0 = np.ascontiguousarray(np.unique(pc, axis=0), dtype=np.int32)
        self.n0 = self.coords0.shape[0]
        self.map0 = be.upload_coords(self.coords0)
        self.latent = be.upload(rng.standard_normal((self.n0, self.LATENT), dtype=np.float32))

        rnd, small = random_weights(be, rng)

        C = self.CHANNELS
        self.w_in, self.b_in = rnd((C[0], self.LATENT), self.LATENT), small(C[0])
        self.blocks = []
        for lv, nb in enumerate(self.BLOCKS):
            c = C[lv]
            self.blocks.append([(rnd((c, 27, c), 27 * c), small(c), small(c, one=True), small(c),
                                 rnd((4 * c, c), c), small(4 * c), rnd((c, 4 * c), 4 * c), small(c))
                                for _ in range(nb)])
        self.ups = []
        for lv in range(len(C) - 1):
            ci, co = C[lv], C[lv + 1]
            self.ups.append({"ws": rnd((8, ci), ci), "bs": be.keep(np.zeros(8, np.float32)),
                             "g1": small(ci, one=True), "b1": small(ci),
                             "w1": rnd((8 * co, 27, ci), 27 * ci), "c1b": small(8 * co),
                             "w2": rnd((co, 27, co), 27 * co), "c2b": small(co)})
        self.w_out, self.b_out = rnd((self.OUT, C[-1]), C[-1]), small(self.OUT)
        self.stats = None

    def forward(self, marks=False, stats=False):
        """One forward; with marks, HIP events 0.. at the stage boundaries; with stats, the per-level sizes
        (read back from the device: the host waits, so those forwards are not the timed ones)."""
        be = self.be
        C = self.CHANNELS
        ev = iter(range(16))
        names = []

        def mark(name):
            if marks:
                be.event(next(ev))
                names.append(name)

        stat_rows = []
        mark("start")
        n = self.n0
        h = be.alloc(n * C[0])
        be.linear(self.latent, self.w_in, self.b_in, h, n, self.LATENT, C[0])
        dmap = self.map0
        rb = be.build_rulebook_for_c2s_map(dmap)
        mark("from_latent")
        owned = None  # the current level's map when an up-block made it
        for lv, c in enumerate(C):
            pairs = be.rulebook_stats(rb)["pairs"] if stats else 0
            for p in self.blocks[lv]:
                out = be.alloc(n * c)
                be.convnext_block(rb, h, *p, out, c, 1e-6)
                h.free()
                h = out
            mark(f"level{lv}_convnext")
            stat_rows.append({"channels": c, "voxels": int(n), "pairs": int(pairs), "convnext_blocks": len(self.blocks[lv])})
            if lv == len(C) - 1:
                break
            u, co = self.ups[lv], C[lv + 1]
            subdiv = be.alloc(n * 8)
            be.linear(h, u["ws"], u["bs"], subdiv, n, c, 8)
            cmap = be.build_c2s_map_device(subdiv, n, coords_map=dmap)
            m = cmap.n
            crb = be.build_rulebook_for_c2s_map(cmap)
            norm1, conv1 = be.alloc(n * c), be.alloc(n * 8 * co)
            be.row_norm(h, u["g1"], u["b1"], norm1, n, c, 1e-6, silu=True)
            be.conv(rb, norm1, u["w1"], u["c1b"], conv1, c, 8 * co)
            h_up, skip, norm2, out = be.alloc(m * co), be.alloc(m * co), be.alloc(m * co), be.alloc(m * co)
            be.c2s_gather_device(conv1, cmap, h_up, co)
            be.skip_repeat_device(h, cmap, skip, c, co)
            be.row_norm(h_up, None, None, norm2, m, co, 1e-6, silu=True)
            if co % 128 == 0:
                be.conv_add(crb, norm2, u["w2"], u["c2b"], skip, out, co, co)
            else:
                conv2 = be.alloc(m * co)
                be.conv(crb, norm2, u["w2"], u["c2b"], conv2, co, co)
                be.add(conv2, skip, out, m * co)
                conv2.free()
            if stats:
                stat_rows[-1]["up_parent_pairs"] = int(pairs)
                stat_rows[-1]["up_child_pairs"] = int(be.rulebook_stats(crb)["pairs"])
            for b in (subdiv, norm1, conv1, h_up, skip, norm2, h):
                b.free()
            rb.free()
            if owned is not None:
                be.free_map(owned)
            h, n, rb, dmap, owned = out, m, crb, cmap, cmap
            mark(f"level{lv}_c2s")
        norm, y = be.alloc(n * C[-1]), be.alloc(n * self.OUT)
        be.row_norm(h, None, None, norm, n, C[-1], 1e-5)
        be.linear(norm, self.w_out, self.b_out, y, n, C[-1], self.OUT)
        mark("head")
        for b in (norm, y, h):
            b.free()
        rb.free()
        if owned is not None:
            be.free_map(owned)
        if stats:
            self.stats = stat_rows
        if marks:
            self.marks = names

    def flops(self):
        """Convs (2 P Ci Co), the ConvNeXt MLPs and the up-blocks' convs, at the sizes the stats forward read back."""
        C, f = self.CHANNELS, 0.0
        for lv, st in enumerate(self.stats):
            c, n = C[lv], st["voxels"]
            f += st["convnext_blocks"] * (wl.conv_flops(st["pairs"], c, c) + 2 * (2 * n * c * 4 * c))
            if "up_child_pairs" in st:
                co = C[lv + 1]
                f += wl.conv_flops(st["up_parent_pairs"], c, 8 * co) + wl.conv_flops(st["up_child_pairs"], co, co)
        return f


class Encoder:
    """The whole shape encoder of the sparse U-Net VAE at the reference's widths, through the backend's entry
    points in the executor's order (src/architectures/sparse_unet_encoder/weights.c:257-262: channels
    {64, 128, 256, 512, 1024}, ConvNeXt blocks {0, 4, 8, 16, 4}, 6 input and 32 latent channels;
    executor.c:160-360 and 392-649):
      input_layer linear 6 -> 64 and the rulebook on the input voxels;
      per level its ConvNeXt blocks (trellis_sparse_hip_convnext_block), then, below the last level, an S2C
      down-block to the next width: row_norm_silu -> conv(Ci -> Co / 8) on the fine voxels -> s2c_build_device
      -> s2c_pack_device and s2c_skip_mean_device -> build_rulebook_for_c2s_map on the coarse voxels ->
      row_norm_silu (no affine) -> conv(Co -> Co) + the skip as one trellis_sparse_hip_conv_add;
      the output head: row_norm (eps 1e-5, no affine) -> to_latent linear 1024 -> 64 (executor.c:551-596: the
      latent is the first 32 channels).
    Input voxels: the config-4 shell set (R = 1024, 3.79M voxels), 6 random channels; random weights per layer.
    """

    CHANNELS = (64, 128, 256, 512, 1024)
    BLOCKS = (0, 4, 8, 16, 4)
    IN = 6
    LATENT = 32

    def __init__(self, be):
        self.be = be
        rng = np.random.default_rng(23)
        self.coords0 = np.ascontiguousarray(wl.make_coords(4), dtype=np.int32)
        self.n0 = self.coords0.shape[0]
        self.map0 = be.upload_coords(self.coords0)
        self.x = be.upload(rng.standard_normal((self.n0, self.IN), dtype=np.float32))

        rnd, small = random_weights(be, rng)

        C = self.CHANNELS
        self.w_in, self.b_in = rnd((C[0], self.IN), self.IN), small(C[0])
        self.blocks = []
        for lv, nb in enumerate(self.BLOCKS):
            c = C[lv]
            self.blocks.append([(rnd((c, 27, c), 27 * c), small(c), small(c, one=True), small(c),
                                 rnd((4 * c, c), c), small(4 * c), rnd((c, 4 * c), 4 * c), small(c))
                                for _ in range(nb)])
        self.downs = []
        for lv in range(len(C) - 1):
            ci, co = C[lv], C[lv + 1]
            self.downs.append({"g1": small(ci, one=True), "b1": small(ci),
                               "w1": rnd((co // 8, 27, ci), 27 * ci), "c1b": small(co // 8),
                               "w2": rnd((co, 27, co), 27 * co), "c2b": small(co)})
        self.w_out, self.b_out = rnd((2 * self.LATENT, C[-1]), C[-1]), small(2 * self.LATENT)
        self.stats = None

    def forward(self, marks=False, stats=False):
        """One forward; with marks, HIP events 0.. at the stage boundaries; with stats, the per-level sizes
        (read back from the device: the host waits, so those forwards are not the timed ones)."""
        be = self.be
        C = self.CHANNELS
        ev = iter(range(16))
        names = []

        def mark(name):
            if marks:
                be.event(next(ev))
                names.append(name)

        stat_rows = []
        mark("start")
        n = self.n0
        h = be.alloc(n * C[0])
        be.linear(self.x, self.w_in, self.b_in, h, n, self.IN, C[0])
        dmap = self.map0
        rb = be.build_rulebook_for_c2s_map(dmap)
        mark("input_layer")
        owned = None  # the current level's map when a down-block made it
        for lv, c in enumerate(C):
            pairs = be.rulebook_stats(rb)["pairs"] if stats else 0
            for p in self.blocks[lv]:
                out = be.alloc(n * c)
                be.convnext_block(rb, h, *p, out, c, 1e-6)
                h.free()
                h = out
            mark(f"level{lv}_convnext")
            stat_rows.append({"channels": c, "voxels": int(n), "pairs": int(pairs), "convnext_blocks": len(self.blocks[lv])})
            if lv == len(C) - 1:
                break
            d, co = self.downs[lv], C[lv + 1]
            norm1, conv1 = be.alloc(n * c), be.alloc(n * (co // 8))
            be.row_norm(h, d["g1"], d["b1"], norm1, n, c, 1e-6, silu=True)
            be.conv(rb, norm1, d["w1"], d["c1b"], conv1, c, co // 8)
            fmap, cmap = be.s2c_build_device(coords_map=dmap)
            m = cmap.n
            packed, skip, norm2, out = be.alloc(m * co), be.alloc(m * co), be.alloc(m * co), be.alloc(m * co)
            be.s2c_pack_device(conv1, fmap, packed, co)
            be.s2c_skip_mean_device(h, fmap, skip, c, co)
            crb = be.build_rulebook_for_c2s_map(cmap)
            be.row_norm(packed, None, None, norm2, m, co, 1e-6, silu=True)
            be.conv_add(crb, norm2, d["w2"], d["c2b"], skip, out, co, co)
            if stats:
                stat_rows[-1]["down_fine_pairs"] = int(pairs)
                stat_rows[-1]["down_coarse_pairs"] = int(be.rulebook_stats(crb)["pairs"])
            for b in (norm1, conv1, packed, skip, norm2, h):
                b.free()
            rb.free()
            be.free_map(fmap)
            if owned is not None:
                be.free_map(owned)
            h, n, rb, dmap, owned = out, m, crb, cmap, cmap
            mark(f"level{lv}_s2c")
        norm, y = be.alloc(n * C[-1]), be.alloc(n * 2 * self.LATENT)
        be.row_norm(h, None, None, norm, n, C[-1], 1e-5)
        be.linear(norm, self.w_out, self.b_out, y, n, C[-1], 2 * self.LATENT)
        mark("to_latent")
        for b in (norm, y, h):
            b.free()
        rb.free()
        if owned is not None:
            be.free_map(owned)
        if stats:
            self.stats = stat_rows
        if marks:
            self.marks = names

    def flops(self):
        """Convs (2 P Ci Co), the ConvNeXt MLPs and the down-blocks' convs, at the sizes the stats forward read
        back."""
        C, f = self.CHANNELS, 0.0
        for lv, st in enumerate(self.stats):
            c, n = C[lv], st["voxels"]
            f += st["convnext_blocks"] * (wl.conv_flops(st["pairs"], c, c) + 2 * (2 * n * c * 4 * c))
            if "down_coarse_pairs" in st:
                co = C[lv + 1]
                f += wl.conv_flops(st["down_fine_pairs"], c, co // 8) + wl.conv_flops(st["down_coarse_pairs"], co, co)
        return f


def run_model(args, kind):
    be = sh.Backend(0, sh.BF16)
    log(f"bench: building the {kind}'s random weights")
    net = Decoder(be) if kind == "decoder" else Encoder(be)
    log(f"bench: {kind} from {net.n0} voxels")
    for _ in range(max(1, args.warmup)):
        net.forward()
    be.synchronize()
    net.forward(stats=True)  # sizes
    be.synchronize()
    net.forward(marks=True)  # the stage split, from a forward with no read-backs of its own
    be.synchronize()
    split = {net.marks[i]: round(be.elapsed(i - 1, i), 3) for i in range(1, len(net.marks))}
    be.synchronize()
    be.event(14)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        net.forward()
    be.event(15)
    be.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    dev = be.elapsed(14, 15) / args.steps
    ms = max(dev, wall)
    data = ("synthetic (config-3 parent shell reduced to R = 64 as the latent voxels; random weights per layer; "
            "subdivision from random logits)" if kind == "decoder" else
            "synthetic (config-4 shell set, R = 1024, as the input voxels; 6 random input channels; random weights "
            "per layer)")
    print(json.dumps({"bench": kind, "dtype": "bf16", "data": data,
                      "steps": args.steps, "warmup": max(1, args.warmup), "ms_per_forward": round(ms, 3),
                      "device_ms_per_forward": round(dev, 3), "wall_ms_per_forward": round(wall, 3),
                      "effective_tflops": round(net.flops() / (ms * 1e-3) / 1e12, 1),
                      "levels": net.stats, "stage_ms": split}))
    be.destroy()


def run_block(args):
    be = sh.Backend(0, sh.BF16)
    job = Block(be, args.block, slots=args.slots, channels=args.channels)
    for _ in range(args.warmup):
        job.step()
    be.synchronize()
    slot_ms = [0.0] * len(job.slots)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        job.step()
        be.synchronize()
        for i in range(len(job.slots)):
            slot_ms[i] += be.elapsed(i, i + 1)
    wall = (time.perf_counter() - t0) * 1e3 / args.steps
    slots = {name: round(ms / args.steps, 4) for name, ms in zip(job.slots, slot_ms)}
    dev = sum(slots.values())
    out = {"block": args.block, "epilogues": "slots" if args.slots else "fused where they apply",
           "dtype": "bf16", "data": "synthetic (config-3 voxel sets, seeded random weights)",
           "steps": args.steps, "warmup": args.warmup, "ms_per_block": round(dev, 4),
           "wall_ms_per_block": round(wall, 4), "effective_tflops": round(job.flops() / (dev * 1e-3) / 1e12, 2),
           "slot_ms": slots}
    if args.block == "mesh":
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as orc

        t0 = time.perf_counter()
        rc, _, faces = orc.fdg_mesh(job.coords, sh.storage_round(job.logits7, be.dtype), 512)
        cpu_ms = (time.perf_counter() - t0) * 1e3
        assert rc == 0 and faces.shape[0] == job.faces
        out.pop("effective_tflops")
        out.update({"voxels": int(job.n), "faces": int(job.faces),
                    "mvoxels_per_s": round(job.n / (dev * 1e-3) / 1e6, 1), "cpu_oracle_ms": round(cpu_ms, 2),
                    "cpu_note": "oracle/trellis_oracle.c orc_fdg_mesh (1 thread), same voxels and logits",
                    "timed": "whole call: corner lookup map, vertices, faces, download of both arrays"})
    elif args.block == "s2c":
        sys.path.insert(0, os.path.join(ROOT, "tests"))
        import oracle_lib as orc

        t0 = time.perf_counter()
        rc, coarse, _, _ = orc.s2c_map(job.fine_coords)
        cpu_ms = (time.perf_counter() - t0) * 1e3
        assert rc == 0 and coarse.shape[0] == job.m
        map_ms = slots["s2c_build_device"]
        out.update({"fine_voxels": int(job.n), "coarse_voxels": int(job.m), "fine_pairs": int(job.fpairs),
                    "coarse_pairs": int(job.pairs), "ci": job.ci, "co": job.co,
                    "s2c_map_mvoxels_per_s": round(job.n / (map_ms * 1e-3) / 1e6, 1),
                    "s2c_map_cpu_oracle_ms": round(cpu_ms, 2),
                    "s2c_map_cpu_note": "oracle/trellis_oracle.c orc_s2c_map (qsort, 1 thread), same fine voxels"})
    elif args.block in ("convnext", "convnext_fused", "convnext_block"):
        out.update({"voxels": int(job.n), "pairs": int(job.pairs), "channels": job.c})
    else:
        out.update({"parents": int(job.n), "children": int(job.m), "parent_pairs": int(job.ppairs),
                    "child_pairs": int(job.pairs), "ci": job.ci, "co": job.co})
    print(json.dumps(out))
    be.destroy()


def conv_schedule(dtype, ci, co, algo):
    """Name of the conv kernel the backend runs (its fallback rules)."""
    mfma = dtype != sh.F32 and ci % 32 == 0 and co % 64 == 0
    if algo in (sh.CONV_AUTO, sh.CONV_COMPACT) and mfma and ci == 64 and co == 64:
        return "os64"  # output-stationary kernel over the compact lists (no fused epilogue)
    if algo in (sh.CONV_AUTO, sh.CONV_COMPACT) and mfma and co % 256 == 0 and ci % 128 == 0:
        return "compact256"  # 256-channel blocks over half map tiles
    if algo in (sh.CONV_AUTO, sh.CONV_COMPACT) and mfma and co % 128 == 0 and ci % 128 == 0 and ci % 256 != 0:
        return "compact_half"  # 4-step units: half map tiles, 4 wavefronts, two blocks per CU
    if algo in (sh.CONV_AUTO, sh.CONV_COMPACT) and mfma and (ci % 128 == 0 or ci == 64):
        return "compact"
    if algo in (sh.CONV_AUTO, sh.CONV_COMPACT, sh.CONV_MASKED) and mfma:
        return "masked"
    return "generic"


def host_cpu_model():
    """The host's CPU model string (/proc/cpuinfo), or the machine name."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


# Every stride-th output row of the CPU baseline's conv (about 5-30 s of CPU
# work per configuration; config 1 runs in full).
CPU_STRIDE = {1: 1, 2: 16, 3: 16, 4: 16, 5: 32}


def cpu_baseline(cfg, w, stride):
    """Single-threaded CPU oracle on a bounded sample of the same workload."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as orc

    dt = wl.CONFIGS[cfg]["dtype"]
    rnd = (lambda a: sh.storage_round(a, dt))
    t = {}
    if cfg == 3:
        t0 = time.perf_counter()
        rc, cc, pp, ss = orc.c2s_map(w["parent_coords"], w["logits"])
        t["subdivide"] = time.perf_counter() - t0
        coords = cc
        t0 = time.perf_counter()
        feats = orc.skip_repeat(rnd(w["parent_feats"]), pp, ss, w["ci"], w["ci"])
        t["broadcast"] = time.perf_counter() - t0
    else:
        coords = w["coords"]
        feats = rnd(w["feats"])
    n = coords.shape[0]
    t0 = time.perf_counter()
    rb = orc.Rulebook(coords)
    t["hash"] = time.perf_counter() - t0
    nbr = rb.neighbors()
    pairs_total = int((nbr >= 0).sum())
    rows = (0, n, stride)
    pairs_sample = int((nbr[::stride] >= 0).sum())
    convs = 2 if cfg == 2 else 1
    t0 = time.perf_counter()
    rb.conv(feats, rnd(w["weight"]), None, w["ci"], w["co"], rows=rows)
    t_sample = time.perf_counter() - t0
    t["conv"] = convs * t_sample * pairs_total / max(1, pairs_sample)
    total = sum(t.values())
    flops = convs * wl.conv_flops(pairs_total, w["ci"], w["co"])
    full = "subdivide, broadcast and hash" if cfg == 3 else "hash"
    conv_part = ("conv on every output row" if stride == 1 else
                 f"conv timed on every {stride}th output row ({pairs_sample} of {pairs_total} pairs) and "
                 "extrapolated by pair count")
    sample = f"cfg{cfg}: {full} on the full set, {conv_part}" + ("; both convs" if convs == 2 else "") + "; 1 thread"
    return {"value": flops / total / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port", "sample": sample,
            "seconds_full_estimate": round(total, 3), "stage_seconds": {k: round(v, 4) for k, v in t.items()},
            "host_cpu": host_cpu_model(), "host_nproc": os.cpu_count()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # The GPU's clocks ramp up over the first few tens of milliseconds of
    # work (config 3's conv: 1.82 ms on the first launch, 1.60 ms from about
    # the 17th), so the default warmup covers that ramp.
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-stride", type=int, default=0,
                    help="every n-th output row for the CPU baseline's conv (default: per configuration)")
    ap.add_argument("--conv-algo", type=int, default=sh.CONV_AUTO)
    ap.add_argument("--block", choices=["convnext", "convnext_fused", "convnext_block", "c2s", "s2c", "mesh"],
                    help="instead of the configuration step, time one decoder block composed from the backend's "
                         "slots at config-3 scale and print its own JSON line")
    ap.add_argument("--channels", type=int, default=128, choices=[128, 256, 512],
                    help="ConvNeXt blocks: 128 on the config-3 children, 256 on its parents, 512 on theirs")
    ap.add_argument("--slots", action="store_true",
                    help="config 2 and the c2s / s2c blocks: run conv -> row_norm_silu and conv -> add as separate "
                         "slots instead of the convs with fused epilogues")
    ap.add_argument("--decoder", action="store_true",
                    help="instead of the configuration step, time the whole shape decoder at the reference's widths "
                         "(5 levels, 32 ConvNeXt blocks, 4 up-blocks) and print its own JSON line")
    ap.add_argument("--encoder", action="store_true",
                    help="instead of the configuration step, time the whole shape encoder at the reference's widths "
                         "(5 levels, 32 ConvNeXt blocks, 4 S2C down-blocks) from the config-4 voxels and print its "
                         "own JSON line")
    ap.add_argument("--calibrate", action="store_true",
                    help="run one fp32 add over 2 x 64Mi-element inputs (512 MiB read, 256 MiB written) so PMC "
                         "byte counters can be scaled against a streaming kernel of known traffic")
    args = ap.parse_args()
    if args.calibrate:
        if sh.device_count() < 1:
            print("bench.py: no HIP device visible", file=sys.stderr)
            sys.exit(1)
        count = 64 * 1024 * 1024
        be = sh.Backend(0, sh.F32)
        a = be.upload(np.ones(count, np.float32))
        b = be.upload(np.ones(count, np.float32))
        y = be.alloc(count)
        be.add(a, b, y, count)
        be.synchronize()
        print(json.dumps({"calibration": "k_add<0>", "read_bytes": 2 * count * 4, "write_bytes": count * 4}))
        be.destroy()
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(more than one GPU is a design only: the sharding of the path is not built)", file=sys.stderr)
        sys.exit(2)
    if sh.device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    if args.decoder:
        return run_model(args, "decoder")
    if args.encoder:
        return run_model(args, "encoder")
    if args.block is not None:
        run_block(args)
        return

    cfg = args.config
    spec = wl.CONFIGS[cfg]
    log(f"bench: generating cfg{cfg} ({spec['name']})")
    w = wl.workload(cfg)
    be = sh.Backend(0, spec["dtype"], conv_algo=args.conv_algo)
    job = Cfg2(be, w, slots=args.slots) if cfg == 2 else {3: Cfg3}.get(cfg, ConvOnly)(be, w)
    log(f"bench: {job.describe()}")
    for _ in range(args.warmup):
        job.step()
    be.synchronize()
    # Timed steps: the production path, without stage events.
    t0 = time.perf_counter()
    be.event(0)
    for _ in range(args.steps):
        job.step()
    be.event(1)
    be.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    dev_ms = be.elapsed(0, 1)
    # Stage breakdown and the conv's launch time (the roofline's denominator):
    # a second pass of as many steps with stage events around each stage.
    be.profile(True)
    be.profile_read(reset=True)
    for _ in range(args.steps):
        job.step()
    be.synchronize()
    stages = be.profile_read(reset=True)
    be.profile(False)
    ms_per_step = max(dev_ms, wall) / args.steps
    flops = job.flops()
    conv_ms, conv_launches = stages["conv"]
    conv_avg = conv_ms / max(1, conv_launches)
    per_launch_flops = wl.conv_flops(job.pairs, job.ci, job.co)
    achieved = per_launch_flops / (conv_avg * 1e-3) / 1e12 if conv_avg > 0 else 0.0
    hm_ms = (stages["hash"][0] + stages["map"][0]) / args.steps
    # Hash + kernel map against HBM: the work definition's bytes (hash 28 N,
    # map 16 N + 108 N + 8 P + 216, the 108 N being an [N][27] neighbour
    # table), and the bytes the production build moves, which writes row
    # masks and per-tile pair lists instead of that table (hash 28 N; map
    # 16 N coordinates + 4 N masks + 5 P pairs (a 4-byte source row and a
    # 1-byte destination row within the tile) + 2 x 108 bytes per 256-row
    # tile of counts and list starts).
    hm_def_bytes = wl.hash_bytes(job.m) + wl.map_bytes(job.m, job.pairs)
    tiles = (job.m + 255) // 256
    hm_moved_bytes = 28.0 * job.m + 16.0 * job.m + 4.0 * job.m + 5.0 * job.pairs + 216.0 * tiles
    hm_gbs = hm_def_bytes / (hm_ms * 1e-3) / 1e9 if hm_ms > 0 else 0.0
    elem = 4 if spec["dtype"] == sh.F32 else 2
    # The conv's binding roofline: compute (2 P Ci Co at the dtype's MFMA or
    # fp32 peak) or HBM (compulsory bytes at 8 TB/s), whichever takes longer.
    conv_bytes = wl.conv_bytes(job.m, job.ci, job.co, elem)
    peak_flops = PEAK_TFLOPS[spec["dtype"]]
    hbm_bound = conv_bytes / (PEAK_HBM_GBS * 1e9) > per_launch_flops / (peak_flops * 1e12)
    if hbm_bound:
        roof_achieved = conv_bytes / (conv_avg * 1e-3) / 1e9 if conv_avg > 0 else 0.0
        roof_peak, roof_unit, roof_bound = PEAK_HBM_GBS, "GB/s", "hbm"
    else:
        roof_achieved, roof_peak, roof_unit, roof_bound = achieved, peak_flops, "TFLOP/s", "mfma"
    # HBM bytes per conv launch come from the committed, copy-calibrated
    # rocprofv3 FETCH_SIZE / WRITE_SIZE summary for this workload and schedule.
    algo_name = conv_schedule(spec["dtype"], job.ci, job.co, args.conv_algo)
    traffic = None
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            entry = json.load(f).get(spec["name"], {}).get(algo_name)
        if entry is not None:
            traffic = round(entry["hbm_bytes_per_launch"])
    except (OSError, ValueError):
        traffic = None
    result = {
        "metric": METRIC,
        "value": round(flops / (ms_per_step * 1e-3) / 1e12, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl.DTYPE_NAMES[spec["dtype"]],
        "data": "synthetic (seeded generator, random-init weights)",
        "config": job.describe(),
        "hash_map_mvoxels_per_s": round(job.m / (hm_ms * 1e-3) / 1e6, 1) if hm_ms > 0 else None,
        "hash_map_roofline": {
            "bound": "hbm", "achieved": round(hm_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(hm_gbs / PEAK_HBM_GBS, 4), "ms_per_step": round(hm_ms, 4),
            "definition_bytes": hm_def_bytes, "moved_bytes": hm_moved_bytes,
            "moved_gbs": round(hm_moved_bytes / (hm_ms * 1e-3) / 1e9, 1) if hm_ms > 0 else 0.0,
        },
        "conv_kernel_tflops": round(achieved, 2),
        "stage_ms_per_step": {k: round(v[0] / args.steps, 4) for k, v in stages.items()},
        "roofline": {
            "bound": roof_bound,
            "kernel": "sparse_conv3d",
            "achieved": round(roof_achieved, 2),
            "peak": roof_peak,
            "unit": roof_unit,
            "frac": round(roof_achieved / roof_peak, 4),
            "traffic": traffic,
            "algorithmic_bytes": conv_bytes,
            "algorithmic_flops": per_launch_flops,
            "schedule": algo_name,
            "avg_launch_ms": round(conv_avg, 4),
        },
        "timing": {"device_event_ms": round(dev_ms, 3), "wall_ms": round(wall, 3),
                   "stages": "stage_ms_per_step and the conv launch time come from a second pass of as many steps "
                             "with stage events (every stage on the backend stream)"},
    }
    if not args.no_cpu_baseline:
        log("bench: timing the CPU oracle baseline")
        result["cpu_baseline"] = cpu_baseline(cfg, w, args.cpu_stride or CPU_STRIDE[cfg])
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    be.destroy()


if __name__ == "__main__":
    main()
