#!/usr/bin/env python3
"""Benchmark of MALOQ's equivariant message-passing hot path on one MI355X.

Headline workload: the reference benchmark's config 2 (32 molecules x 40
atoms, ~30k directed edges, lmax 4, mmax 2, 128 channels, 8 Gaussian RBFs).
A step is one fused message block, forward and backward, with inputs already
resident in HBM: per-edge Euler angles + Wigner-D, the radial MLP (fused HIP), the
fused rotate -> SO(2) -> inverse-rotate -> segment-sum kernel, and its input,
radial and weight gradients.  `value` is edges per second, in fp32 by default
(the reference's path computes in fp32, esen_osh.py:277-281).

The JSON line also carries the roofline of the dominant kernel (the fused
forward launch, MFMA-bound), the CPU baseline (the build's own CPU
restatement of the reference's PyTorch path, timed on a bounded sample), and
one object per other configuration of the benchmark, each with its own
throughput, roofline and CPU baseline: config 2 in the other precision,
config 1 (rotation round trip, HBM-bound), configs 4 and 5 (fused block,
bf16), config 3 and config 5's basis transforms (H-blocks/s, with and without
the per-structure row plan), the edge-degree embedding and the
two-convolution Edgewise block.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--dtype fp32|bf16]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

PEAK_BF16 = 2.5e15      # dense MFMA, MI355X
PEAK_FP32 = 157.3e12
PEAK_HBM = 8.0e12


def fused_flops_per_edge(L, M, c_in, c_out):
    """Algorithmic FLOPs of rotate -> SO(2) -> inverse rotate -> scatter per edge."""
    rot = sum(min(2 * l + 1, 2 * M + 1) * (2 * l + 1) for l in range(L + 1))
    mac = (L + 1) ** 2 * c_in * c_out + sum(4 * (L - m + 1) ** 2 * c_in * c_out for m in range(1, M + 1))
    return 2 * (rot * c_in + mac + rot * c_out) + (L + 1) ** 2 * c_out


def make_radial(n_rbf, hidden, out, device):
    """RadialMLP([n_rbf, hidden, hidden, out]) (radial.py:115-142), fused HIP kernels."""
    from maloq_amd.radial import RadialMLP
    return RadialMLP([n_rbf, hidden, hidden, out]).to(device)


_RBF: dict = {}


def gaussian_rbf(dist, start, stop, num):
    """Gaussian smearing of the edge lengths.  The offsets and the coefficient
    are made once per (start, stop, num, device), as a smearing module makes
    them at construction: reading the coefficient back from the device on every
    step would stall the step on the GPU."""
    import torch
    key = (start, stop, num, str(dist.device))
    if key not in _RBF:
        off = torch.linspace(start, stop, num)  # host tensor: no device read
        _RBF[key] = (off.to(dist.device), -0.5 / (off[1] - off[0]).item() ** 2)
    offset, coeff = _RBF[key]
    return torch.exp(coeff * (dist.view(-1, 1) - offset.view(1, -1)) ** 2)


# message-block legs: (graph loader, lmax, mmax, channels, gated, RBF cutoff)
MESSAGE_CONFIGS = {
    "config1": ("config1_graph", 2, 2, 32, False, 5.0),
    "config2": ("config2_graph", 4, 2, 128, False, 6.0),
    "config4": ("config4_graph", 6, 2, 128, True, 8.0),
    "config5": ("config5_graph", 4, 2, 256, False, 6.0),
}
_GRAPHS: dict = {}


def _graph(name):
    from maloq_amd import synth
    if name not in _GRAPHS:
        _GRAPHS[name] = getattr(synth, name)()
    return _GRAPHS[name]


def message_workload(dtype_name, seed=0, cfg="config2"):
    """Tensors of a message-block configuration on cuda:0 (default config 2)."""
    import numpy as np
    import torch
    from maloq_amd import message as M

    dev = torch.device("cuda:0")
    dt = {"bf16": torch.bfloat16, "fp32": torch.float32}[dtype_name]
    gname, L, Mm, C, gate, cutoff = MESSAGE_CONFIGS[cfg]
    g = _graph(gname)
    gen = torch.Generator().manual_seed(seed)
    N, E = g.num_nodes, g.num_edges
    plan = M.MessagePlan(torch.from_numpy(np.stack([g.src, g.dst])).to(dev), N)
    vec = plan.sort_edges(torch.from_numpy(g.edge_distance_vec()).float().to(dev))
    dist = vec.norm(dim=1)
    x = torch.randn(N, (L + 1) ** 2, C, generator=gen).to(device=dev, dtype=dt).requires_grad_()
    k0 = (L + 1) * C
    extra = L * C if gate else 0
    w0 = (torch.randn((L + 1) * C + extra, k0, generator=gen) / math.sqrt(k0)).to(dev).requires_grad_()
    b0 = torch.zeros((L + 1) * C + extra, device=dev, requires_grad=True)
    wm = []
    for m in range(1, Mm + 1):
        k = (L - m + 1) * C
        wm.append((torch.randn(2 * (L - m + 1) * C, k, generator=gen) / math.sqrt(k)).to(dev).requires_grad_())
    torch.manual_seed(seed)
    radial = make_radial(8, 64, M.rad_width(L, Mm, C), dev)
    gout = torch.randn(N, (L + 1) ** 2, C, generator=gen).to(dev)
    return dict(graph=g, plan=plan, vec=vec, dist=dist, x=x, w0=w0, b0=b0, wm=wm, radial=radial,
                gout=gout, L=L, M=Mm, C=C, dt=dt, N=N, E=E, gate=gate, cutoff=cutoff, cfg=cfg)


def message_step(w, backward=True, ops=True):
    """One training step of the fused block: Euler angles, radial MLP, the
    block (through the module path, or with ``ops`` through the registered
    C++ operators maloq_hip::message_block_fwd / _bwd; same kernels and bits)."""
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    block = M.message_block
    if ops:
        from maloq_amd import ops as O
        block = O.message_block
    eul = extract_euler_angles(w["vec"], seed=1234)
    rad = w["radial"](gaussian_rbf(w["dist"], 0.0, w["cutoff"], 8), out_dtype=w["dt"])
    out = block(w["x"], w["plan"], eul, rad, w["w0"], w["b0"], w["wm"], w["L"], w["M"], gate=w["gate"])
    if backward:
        # a training step starts from cleared gradients (zero_grad(set_to_none=True))
        for t in [w["x"], w["w0"], w["b0"], *w["wm"], *w["radial"].parameters()]:
            t.grad = None
        out.backward(w["gout"])
    return out


def fock_head_leg(reps=10):
    """Fock_Irreps_Head (esen_osh.py:522-1064) forward, and forward + backward,
    on the config-3 batch (64 molecules; lmax 4 node and edge embeddings of
    width C = 128, the reference's model width), and the label-side eval
    formats on the same batch: the padding mask, sort_by_m of one molecule's
    Fock matrix, and the CSR export of the whole block list."""
    import numpy as np
    import torch
    from maloq_amd import synth
    from maloq_amd.fock_utils import create_label_unpadding_mask, sort_by_m, sparse_block_matrix_to_csr_arrays
    from maloq_amd.irreps_head import Fock_Irreps_Head
    from maloq_amd.matrix2labels import SparseBlockMatrix
    bw = basis_workload()
    t, dev, T = bw["tables"], bw["data"].device, bw["T"]
    Z, rows, cols = bw["Z"], bw["rows"], bw["cols"]
    off_site = rows != cols
    src, dst = rows[off_site], cols[off_site]
    N, E = len(Z), int(off_site.sum())
    lmax, C = 4, 128
    torch.manual_seed(0)
    head = Fock_Irreps_Head("+".join(f"{C}x{l}e" for l in range(lmax + 1)), t.req_output_irreps, lmax, C,
                            ls_list=t.ls_list).to(dev)
    d = (lmax + 1) ** 2
    emb = {"node_embeddings": torch.randn(N, d, C, device=dev, requires_grad=True),
           "edge_embeddings": torch.randn(E, d, C, device=dev, requires_grad=True)}

    def fwd():
        with torch.no_grad():
            return head(emb, None)
    node, edge = fwd()
    gn, ge = torch.randn_like(node), torch.randn_like(edge)

    def step():
        n_, e_ = head(emb, None)
        torch.autograd.backward([n_, e_], [gn, ge])
    t_fwd = kernel_time_events(fwd, reps)
    t_step = kernel_time_events(step, reps)
    # the head reads the embeddings and writes the label rows (and the reverse
    # in the backward): its algorithmic bytes per forward
    fwd_bytes = (N + E) * (d * C + T) * 4
    out = {"metric": "label rows/s", "config": f"config 3 batch: {N} atoms, {E} atom pairs, T = {T}, C = {C}",
           "fwd_rows_per_s": (N + E) / t_fwd, "fwd_bwd_rows_per_s": (N + E) / t_step,
           "us_fwd": t_fwd * 1e6, "us_fwd_bwd": t_step * 1e6,
           "roofline": {"scope": "whole forward (per-l linears, gate, column gather)", "bound": "hbm",
                        "achieved": fwd_bytes / t_fwd / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                        "frac": fwd_bytes / t_fwd / PEAK_HBM, "bytes_per_call": fwd_bytes}}
    # padding mask of the batch (host tables + one launch), wall time
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        create_label_unpadding_mask(t.orbital_template, Z, src, dst, T, dev)
    torch.cuda.synchronize()
    out["us_label_mask"] = (time.perf_counter() - t0) / reps * 1e6
    # sort_by_m of the largest molecule's dense Fock matrix
    z, p = max(bw["mols"], key=lambda m: len(m[0]))
    H, _ = synth.dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=0, cutoff=8.0)
    Hd = torch.from_numpy(H.astype(np.float32)).to(dev)
    sort_by_m(Hd, CFG3_BASIS, z)
    ts = kernel_time_events(lambda: sort_by_m(Hd, CFG3_BASIS, z), reps)
    out["sort_by_m"] = {"n": int(H.shape[0]), "us": ts * 1e6, "GBps": 2 * Hd.numel() * 4 / ts / 1e9}
    # CSR arrays of the whole block list (device arrays; the scipy object is a host copy)
    sbm = SparseBlockMatrix(data=bw["data"], block_data_offsets=bw["bdo"],
                            fock_block_rows=torch.from_numpy(rows).to(dev),
                            fock_block_cols=torch.from_numpy(cols).to(dev),
                            fock_block_offsets=torch.from_numpy(bw["off"]).to(dev))
    sparse_block_matrix_to_csr_arrays(sbm)
    tc = kernel_time_events(lambda: sparse_block_matrix_to_csr_arrays(sbm), reps)
    nnz = bw["data"].numel()
    out["csr_export"] = {"nnz": nnz, "us": tc * 1e6,
                         "GBps": (4 * nnz + (4 + 8) * nnz) / tc / 1e9}  # values in, values + column indices out
    del bw, head, emb
    torch.cuda.empty_cache()
    return out


def graph_step_leg(cfg="config1", dtype="fp32", reps=50):
    """The training step of `message_step` (through the operators) enqueued op
    by op, and the same step captured once into a HIP graph (torch.cuda.graph)
    and replayed: wall time per step, host enqueue included.  Small graphs are
    bound by the host's enqueue of the step's ~20 launches; the replay
    enqueues one graph."""
    import torch
    w = message_workload(dtype, cfg=cfg)
    step = lambda: message_step(w, True)
    # everything on one side stream: autograd's gradient accumulators stay on
    # the stream they were made on, and the capture runs after a warm-up there
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        t_eager = time_steps(step, reps, 5)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=s):
            step()
        t_graph = time_steps(graph.replay, reps, 5)
    torch.cuda.current_stream().wait_stream(s)
    E = w["E"]
    del graph, w
    torch.cuda.empty_cache()
    return {"metric": "edges/s (fused block fwd+bwd, wall time)", "cfg": cfg, "dtype": dtype, "edges": E,
            "us_per_step_eager": t_eager * 1e6, "us_per_step_hip_graph": t_graph * 1e6,
            "eager_edges_per_s": E / t_eager, "hip_graph_edges_per_s": E / t_graph}


def time_steps(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps


def kernel_time_events(fn, reps):
    """Average duration of fn's launches, HIP events on the current stream."""
    import torch
    s = torch.cuda.current_stream()
    fn()
    s.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(s)
    for _ in range(reps):
        fn()
    b.record(s)
    b.synchronize()
    return a.elapsed_time(b) / 1e3 / reps


def fused_forward_launch_time(w, reps=20):
    import torch
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    with torch.no_grad():
        eul = extract_euler_angles(w["vec"], seed=1234)
        rad = w["radial"](gaussian_rbf(w["dist"], 0.0, w["cutoff"], 8), out_dtype=w["dt"])
        x = w["x"].detach()
        wpack = M.pack_weights(w["w0"], w["wm"], w["L"], w["M"], w["gate"], w["C"], w["C"], w["dt"], 0)
        f = lambda: M.message_forward(x, w["plan"], eul, rad, w["w0"], w["b0"], w["wm"], w["L"], w["M"],
                                      gate=w["gate"], wpack=wpack)
        return kernel_time_events(f, reps)


def gated_flops_extra(L, c_in, c_out):
    """FLOPs per edge of the gate rows (L c_out extra m = 0 outputs) and the gate itself."""
    return 2 * (L + 1) * c_in * L * c_out + ((L + 1) ** 2 - 1) * c_out


# ---------------------------------------------------------- basis transform
CFG3_BASIS = {1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2], 7: [0, 0, 0, 1, 1, 2], 8: [0, 0, 0, 1, 1, 2]}
# def2-TZVPD shells (src/maloq/fock_utils/basis_sets.py:28) of H/C/N/O, plus Ga
# (4 d shells) and I (2 f shells): the template then has the 64 orbitals of the
# whole dictionary, 4096 label columns, as the OMol loader builds it from every
# element (dataset_utils/get_loader.py:106-107); the molecules are H/C/N/O.
TZVPD_BASIS = {1: [0, 0, 0, 1, 1], 6: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 2],
               7: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 2], 8: [0, 0, 0, 0, 0, 1, 1, 1, 2, 2, 3, 0, 1, 2],
               31: [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 2, 3, 0, 2],
               53: [0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 2, 2, 2, 3, 3, 0, 1, 2]}


def basis_workload(basis=None):
    """Config 3 as one block list (all on-site + off-site < 8 A blocks of 64
    molecules), so the whole batch is one launch; ``basis`` (default: config 3's
    def2-SVP-like one) gives the orbitals and the label template."""
    import numpy as np
    import torch
    from maloq_amd import synth
    from maloq_amd import tensor_decomp as ptd
    from maloq_amd.basis_transform import HipE3TensorDecomp

    dev = torch.device("cuda:0")
    t = ptd.BasisTables(basis or CFG3_BASIS)
    base = ptd.e3TensorDecomp(t.req_output_irreps, t.out_js_list, torch.float32, device_torch=dev)
    hip = HipE3TensorDecomp(base)
    Zs, offs, rows, cols, data = [], [0], [], [], []
    atom0 = 0
    n_bytes = 0
    mols = synth.config3_molecules()
    for m, (z, p) in enumerate(mols):
        H, off = synth.dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=m, cutoff=8.0)
        src, dst, _ = synth.radius_graph(p, 8.0)
        r, c = synth.atom_pair_rows(src, dst, len(z))
        for i, j in zip(r, c):
            blk = H[off[i]:off[i + 1], off[j]:off[j + 1]]
            data.append(blk.reshape(-1))
            n_bytes += 4 * blk.size
        rows.append(r + atom0)
        cols.append(c + atom0)
        Zs.append(z)
        offs.extend((off[1:] + offs[-1]).tolist())
        atom0 += len(z)
    rows = np.concatenate(rows).astype(np.int32)
    cols = np.concatenate(cols).astype(np.int32)
    Z = np.concatenate(Zs).astype(np.int32)
    off = np.asarray(offs, np.int32)
    sizes = np.array([d.size for d in data], np.int64)
    bdo = np.concatenate([[0], np.cumsum(sizes)]).astype(np.int64)
    flat = torch.from_numpy(np.concatenate(data).astype(np.float32)).to(dev)
    return dict(tables=t, hip=hip, base=base, Z=Z, off=off, rows=rows, cols=cols,
                bdo=torch.from_numpy(bdo).to(dev), data=flat, n_blocks=len(rows),
                block_bytes=n_bytes, T=base.in_slices[-1], mols=mols)


def basis_timing(bw, reps=50):
    import torch
    hip, t = bw["hip"], bw["tables"]
    args = (bw["off"], bw["Z"], bw["rows"], bw["cols"], t.orbital_template)
    # upload index arrays once (the dataset's device-resident tables)
    import numpy as np
    dev = bw["data"].device
    dev_args = tuple(torch.as_tensor(np.asarray(a, np.int32), device=dev) for a in args[:4])
    # the row plan (per-structure: block bases and kinds, ordered by kind) is
    # built once, like the message graph's sort; its cost is reported apart
    make = lambda: hip.make_plan(bw["data"], *dev_args, t.orbital_template, block_data_offsets=bw["bdo"])
    plan = make()
    plan_s = kernel_time_events(make, max(1, reps // 5))
    out = hip.fock_to_irreps(bw["data"], *args, block_data_offsets=bw["bdo"])
    fwd = kernel_time_events(lambda: hip.fock_to_irreps(bw["data"], *dev_args, t.orbital_template,
                                                        block_data_offsets=bw["bdo"], plan=plan), reps)
    back = torch.empty_like(bw["data"])
    inv = kernel_time_events(lambda: hip.irreps_to_fock(out, back, *dev_args, t.orbital_template,
                                                        block_data_offsets=bw["bdo"], plan=plan), reps)
    rt = ((back - bw["data"]).abs().max() / bw["data"].abs().max()).item()
    # without a plan: one launch each, the rows described from the pair list
    # inside the kernel (a structure transformed once)
    fwd_pl = kernel_time_events(lambda: hip.fock_to_irreps(bw["data"], *dev_args, t.orbital_template,
                                                           block_data_offsets=bw["bdo"]), reps)
    inv_pl = kernel_time_events(lambda: hip.irreps_to_fock(out, back, *dev_args, t.orbital_template,
                                                           block_data_offsets=bw["bdo"]), reps)
    return fwd, inv, rt, plan_s, fwd_pl, inv_pl


def wide_basis_leg(reps=20, cpu=True):
    """Config 3's molecules under the def2-TZVPD template (4096-column label
    rows, several column groups per row tile): H-blocks/s both directions, with
    a prebuilt plan and from the pair list, HBM roofline of the forward."""
    import torch
    bw = basis_workload(TZVPD_BASIS)
    tf, ti, rt, tplan, tfp, tip = basis_timing(bw, reps)
    nb = bw["n_blocks"]
    bpb = (bw["block_bytes"] + 4 * bw["T"] * nb) / nb
    out = {"metric": "H-blocks/s", "fwd": nb / tf, "inv": nb / ti, "fwd_with_plan": nb / (tf + tplan),
           "inv_with_plan": nb / (ti + tplan), "fwd_pair_list": nb / tfp, "inv_pair_list": nb / tip,
           "blocks": nb, "T": int(bw["T"]), "column_groups": bw["hip"].ngroups, "round_trip_rel_err": rt,
           "plan_ms": tplan * 1e3, "config": "config 3 molecules (64 x 30-50 atoms, H/C/N/O), def2-TZVPD "
                                             "template (4096 columns), block list",
           "roofline": {"kernel": "transform_kernel<FOCK,ROWS> (block list, column groups)", "bound": "hbm",
                        "achieved": bpb * nb / tf / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                        "frac": bpb * nb / tf / PEAK_HBM, "bytes_per_block": bpb,
                        "traffic": load_traffic("fock_to_irreps_tzvpd")}}
    if cpu:
        out["cpu_baseline"] = cpu_basis_baseline(bw, budget_s=10.0)
    del bw
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------- CPU legs
def cpu_message_baseline(budget_s=15.0, cfg="config2"):
    """The build's CPU restatement of the reference path (RadialMLP,
    bmm(wigner), einsum to_m, SO2_Convolution [+ GateActivation], einsum,
    bmm(wigner_inv), index_add_), fp32 torch on the host cores, forward +
    backward, on the in-edges of the first nodes of the configuration (whole
    molecules for configs 2 and 4), sized to about ``budget_s`` of CPU work."""
    import numpy as np
    import torch
    from oracle import message as omsg
    from oracle import rotation as orot
    from maloq_amd import message as M

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    gname, L, Mm, C, gate, cutoff = MESSAGE_CONFIGS[cfg]
    g = _graph(gname)
    gen = torch.Generator().manual_seed(0)
    Jd = orot.load_jd(torch.float32)
    k0 = (L + 1) * C
    extra = L * C if gate else 0
    conv = {"w0": torch.randn(k0 + extra, k0, generator=gen) / math.sqrt(k0),
            "b0": torch.zeros(k0 + extra),
            "wm": [torch.randn(2 * (L - m + 1) * C, (L - m + 1) * C, generator=gen) / math.sqrt((L - m + 1) * C)
                   for m in range(1, Mm + 1)], "c_out": C}
    for k in ("w0", "b0"):
        conv[k].requires_grad_()
    for wmm in conv["wm"]:
        wmm.requires_grad_()
    # the reference's RadialMLP as torch modules (radial.py:115-142), fp32 CPU
    torch.manual_seed(0)
    radial = torch.nn.Sequential(torch.nn.Linear(8, 64), torch.nn.LayerNorm(64), torch.nn.SiLU(),
                                 torch.nn.Linear(64, 64), torch.nn.LayerNorm(64), torch.nn.SiLU(),
                                 torch.nn.Linear(64, M.rad_width(L, Mm, C)))
    x_all = torch.randn(g.num_nodes, (L + 1) ** 2, C, generator=gen)
    # node counts: whole molecules where the graph has them
    unit = int(np.sum(g.mol == 0)) if g.mol.max() > 0 else 10

    def run(n_nodes):
        sel = g.dst < n_nodes
        ei = torch.from_numpy(np.stack([g.src[sel], g.dst[sel]]))
        vec = torch.from_numpy(g.edge_distance_vec()[sel]).float()
        x = x_all.clone().requires_grad_()
        t0 = time.perf_counter()
        rad = radial(gaussian_rbf(vec.norm(dim=1), 0.0, cutoff, 8))
        eul = orot.init_edge_rot_euler_angles(vec, torch.rand(len(vec), generator=gen))
        out = omsg.message_block(x, ei, eul, Jd, L, Mm, conv, rad=rad, gate=gate)
        out.backward(torch.ones_like(out))
        return time.perf_counter() - t0, int(sel.sum())

    run(unit)  # warm-up
    t1, _ = run(unit)
    n = max(1, min(g.num_nodes // unit, int(budget_s / 5 / max(t1, 1e-3)))) * unit
    times = []
    for _ in range(5):
        t, e = run(n)
        times.append(t)
    t = sorted(times)[len(times) // 2]
    return {"value": e / t, "unit": "edges/s", "cores": cores, "kind": "port",
            "sample": f"{cfg}, in-edges of the first {n} nodes ({e} edges), fp32 torch CPU, fwd+bwd, median of 5",
            "threads": torch.get_num_threads(), "cpu": _cpu_model()}


def cpu_basis_baseline(bw, budget_s=8.0):
    """numpy_single_matrix2label restated + dense get_net_out matmul, per molecule."""
    import numpy as np
    import torch
    from oracle import matrix2labels as om2l
    from oracle import tensor_decomp as otd
    from maloq_amd import synth

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t = bw["tables"]
    o = otd.E3TensorDecomp(t.out_js_list, dtype=torch.float32)
    total_blocks, total_t = 0, 0.0
    for m, (z, p) in enumerate(bw["mols"]):
        H, off = synth.dense_hamiltonian(z, p, t.orbitals_per_atom(z), seed=m, cutoff=8.0)
        src, dst, _ = synth.radius_graph(p, 8.0)
        r, c = synth.atom_pair_rows(src, dst, len(z))
        t0 = time.perf_counter()
        lab = np.zeros((len(r), int(bw["T"])), np.float32)
        om2l.single_matrix2label(t.orbital_template, off, z, r, c, H, lab, True)
        o.get_net_out(torch.from_numpy(lab))
        total_t += time.perf_counter() - t0
        total_blocks += len(r)
        if total_t > budget_s:
            break
    return {"value": total_blocks / total_t, "unit": "H-blocks/s", "cores": cores, "kind": "port",
            "sample": f"config 3 molecules, {m + 1} molecule(s) ({total_blocks} blocks), T = {int(bw['T'])}, "
                      f"numpy gather + fp32 matmul"}


# ------------------------------------------------------- config 1: rotation
def rotation_leg(cpu=True):
    """Config 1 (12 atoms, lmax 2, C 32, fp32): x[src] rotated into the edge
    frame and back (two maloq_rotate launches), single launches and a batch of
    round trips captured in one HIP graph; the identity and global-rotation
    errors; and the same kernel at config-2 scale (36 804 edges, lmax 4,
    C 128), where it is HBM-bound, for its roofline."""
    import numpy as np
    import torch
    from maloq_amd import _lib
    from maloq_amd import message as M
    from maloq_amd.rotate import rotate
    from maloq_amd.wigner import extract_euler_angles
    dev = torch.device("cuda:0")
    lib = _lib.load()
    out = {"metric": "edges/s (rotate in + rotate out)"}

    def raw(xdt, odt, L, x, C, gather, E, eul, inv, y):
        rc = lib.maloq_rotate(xdt, odt, L, x.data_ptr(), C, gather.data_ptr() if gather is not None else None, E,
                              eul.data_ptr(), None, M._jd_dev(L, dev).data_ptr(), inv, y.data_ptr(),
                              torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.maloq_last_error()

    g = _graph("config1_graph")
    L, C, E = 2, 32, g.num_edges
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(g.num_nodes, 9, C, generator=gen).to(dev)
    vec = torch.from_numpy(g.edge_distance_vec()).float().to(dev)
    eul = extract_euler_angles(vec, seed=0)
    src = torch.from_numpy(g.src).to(device=dev, dtype=torch.int32)
    y = torch.empty(E, 9, C, device=dev)
    z = torch.empty(E, 9, C, device=dev)

    def rt():
        raw(0, 0, L, x, C, src, E, eul, 0, y)
        raw(0, 0, L, y, C, None, E, eul, 1, z)
    t1 = kernel_time_events(rt, 200)
    nb = 50
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        rt()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            for _ in range(nb):
                rt()
    torch.cuda.current_stream().wait_stream(s)
    tg = kernel_time_events(graph.replay, 20) / nb
    torch.cuda.synchronize()
    ident = ((z - x[src.long()]).abs().max() / x.abs().max()).item()
    out.update({"config": f"config 1: 12 atoms, {E} directed edges (5 A cutoff), lmax 2, 32 channels, fp32",
                "value": E / tg, "edges": E, "us_per_round_trip_single_launches": t1 * 1e6,
                "us_per_round_trip_hip_graph": tg * 1e6, "identity_rel_err": ident})
    # equivariance: m = 0 rows of the edge frame are unchanged by a global rotation
    a, b, c = 0.3, 1.1, -0.7
    from oracle import rotation as orot
    tt = lambda v: torch.tensor([v], dtype=torch.float64)
    R = torch.from_numpy(_yxy(a, b, c))
    Dfull = torch.block_diag(*[orot.wigner_D(l, tt(a), tt(b), tt(c), orot.load_jd())[0] for l in range(3)])
    xr = torch.einsum("ij,njc->nic", Dfull, x.cpu().double()).float().to(dev)
    eul_r = extract_euler_angles((torch.from_numpy(g.edge_distance_vec()) @ R.T).float().to(dev), seed=0)
    y0 = rotate(x, L, eulers=eul, gather=src.long())
    y1 = rotate(xr, L, eulers=eul_r, gather=src.long())
    m0 = [l * l + l for l in range(3)]
    out["equivariance_rel_err_m0_rows"] = ((y1[:, m0] - y0[:, m0]).abs().max() / y0.abs().max()).item()
    # the kernel at config-2 scale: HBM roofline
    g2 = _graph("config2_graph")
    L2, C2, E2 = 4, 128, g2.num_edges
    d2 = 25
    eul2 = extract_euler_angles(torch.from_numpy(g2.edge_distance_vec()).float().to(dev), seed=0)
    src2 = torch.from_numpy(g2.src).to(device=dev, dtype=torch.int32)
    scale = {}
    for name, code, dt in (("fp32", 0, torch.float32), ("bf16", 1, torch.bfloat16)):
        x2 = torch.randn(g2.num_nodes, d2, C2, generator=gen).to(device=dev, dtype=dt)
        y2 = torch.empty(E2, d2, C2, device=dev, dtype=dt)
        z2 = torch.empty(E2, d2, C2, device=dev, dtype=dt)
        es = 2 if code else 4
        t_in = kernel_time_events(lambda: raw(code, code, L2, x2, C2, src2, E2, eul2, 0, y2), 20)
        t_out = kernel_time_events(lambda: raw(code, code, L2, y2, C2, None, E2, eul2, 1, z2), 20)
        b_in = E2 * (2 * d2 * C2 * es + 12 + 4)
        b_out = E2 * (2 * d2 * C2 * es + 12)
        scale[name] = {"rotate_in_us": t_in * 1e6, "rotate_out_us": t_out * 1e6,
                       "edges_per_s_round_trip": E2 / (t_in + t_out),
                       "roofline": {"kernel": "rotate_kernel<4> (rotate in, gather of x[src])", "bound": "hbm",
                                    "achieved": b_in / t_in / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                                    "frac": b_in / t_in / PEAK_HBM, "bytes_per_edge": b_in / E2},
                       "rotate_out_hbm_frac": b_out / t_out / PEAK_HBM}
    out["config2_scale"] = scale
    if cpu:
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        e = eul.cpu()
        xs = x.cpu()
        Jd = orot.load_jd(torch.float32)
        srcl = src.long().cpu()

        def cpu_rt():
            w = orot.eulers_to_wigner((e[:, 0], e[:, 1], e[:, 2]), 0, L, Jd)
            yy = torch.bmm(w, xs[srcl])
            return torch.bmm(w.transpose(1, 2), yy)
        cpu_rt()
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 3.0:
            cpu_rt()
            reps += 1
        out["cpu_baseline"] = {"value": E * reps / (time.perf_counter() - t0), "unit": "edges/s", "cores": cores,
                               "kind": "port", "sample": f"config 1, whole graph ({E} edges), eulers_to_wigner + "
                                                         f"bmm + bmm^T, fp32 torch CPU, {reps} repetitions"}
    return out


def _yxy(a, b, c):
    ca, sa, cb, sb, cc, sc = math.cos(a), math.sin(a), math.cos(b), math.sin(b), math.cos(c), math.sin(c)
    import numpy as np
    Ry = lambda co, si: np.array([[co, 0, si], [0, 1, 0], [-si, 0, co]])
    Rx = np.array([[1, 0, 0], [0, cb, -sb], [0, sb, cb]])
    return Ry(ca, sa) @ Rx @ Ry(cc, sc)


# --------------------------------------------- config 5: block-sparse basis
SIO2_BASIS = {14: [0, 0, 1, 1, 2], 8: [0, 0, 1, 1, 2]}


def sparse_basis_workload():
    """Config 5's 2s2p1d (T = 169) block list over the 2000-atom cell: every atom
    pair within 6 A plus the on-site blocks, N(0, 1) exp(-r / 2), on-site - 10."""
    import numpy as np
    import torch
    from maloq_amd import synth
    from maloq_amd import tensor_decomp as ptd
    from maloq_amd.basis_transform import HipE3TensorDecomp
    from oracle import matrix2labels as om2l
    dev = torch.device("cuda:0")
    g = _graph("config5_graph")
    t = ptd.BasisTables(SIO2_BASIS)
    base = ptd.e3TensorDecomp(t.req_output_irreps, t.out_js_list, torch.float32, device_torch=dev)
    hip = HipE3TensorDecomp(base)
    rows, cols = synth.atom_pair_rows(g.src, g.dst, g.num_nodes)
    off = np.concatenate([[0], np.cumsum(t.orbitals_per_atom(g.Z))]).astype(np.int32)
    bdo = om2l.block_data_offsets(off, rows, cols)
    rng = np.random.default_rng(0)
    data = rng.standard_normal(int(bdo[-1])).astype(np.float32)
    r = np.linalg.norm(g.vec, axis=1)
    n_e = len(g.src)
    sizes = np.diff(bdo)
    data *= np.repeat(np.concatenate([np.exp(-r / 2), np.ones(len(rows) - n_e)]).astype(np.float32), sizes)
    for k in range(n_e, len(rows)):
        i = rows[k]
        n = off[i + 1] - off[i]
        blk = data[bdo[k]:bdo[k + 1]].reshape(n, n)
        blk -= 10.0 * np.eye(n, dtype=np.float32)
    return dict(tables=t, hip=hip, Z=g.Z.astype(np.int32), off=off, rows=rows.astype(np.int32),
                cols=cols.astype(np.int32), bdo=torch.from_numpy(bdo).to(dev), bdo_np=bdo,
                data=torch.from_numpy(data).to(dev), data_np=data, n_blocks=len(rows),
                block_bytes=4 * int(bdo[-1]), T=base.in_slices[-1])


def cpu_sparse_basis_baseline(sw, budget_s=8.0):
    """The restated K13 gather (numpy_single_matrix2label over the block list) +
    get_net_out as an fp32 matmul, on whole-cell row chunks until the budget."""
    import numpy as np
    import torch
    from oracle import matrix2labels as om2l
    from oracle import tensor_decomp as otd
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    t = sw["tables"]
    o = otd.E3TensorDecomp(t.out_js_list, dtype=torch.float32)
    n = sw["n_blocks"]
    step = 4096
    done, tot = 0, 0.0
    while done < n and tot < budget_s:
        sl = slice(done, min(n, done + step))
        rows, cols = sw["rows"][sl], sw["cols"][sl]
        bdo = sw["bdo_np"][sl.start:sl.stop + 1] - sw["bdo_np"][sl.start]
        data = sw["data_np"][sw["bdo_np"][sl.start]:sw["bdo_np"][sl.stop]]
        t0 = time.perf_counter()
        lab = np.zeros((len(rows), sw["T"]), np.float32)
        om2l.single_matrix2label_sparse(t.orbital_template, sw["off"], sw["Z"], rows, cols, data, bdo, lab, True)
        o.get_net_out(torch.from_numpy(lab))
        tot += time.perf_counter() - t0
        done = sl.stop
    return {"value": done / tot, "unit": "H-blocks/s", "cores": cores, "kind": "port",
            "sample": f"config 5, {done} of {n} blocks, numpy block-list gather + fp32 matmul"}


def sparse_basis_leg(sw, reps=30):
    import torch
    hip, t = sw["hip"], sw["tables"]
    dev = sw["data"].device
    import numpy as np
    dev_args = tuple(torch.as_tensor(np.asarray(a, np.int32), device=dev)
                     for a in (sw["off"], sw["Z"], sw["rows"], sw["cols"]))
    make = lambda: hip.make_plan(sw["data"], *dev_args, t.orbital_template, block_data_offsets=sw["bdo"])
    plan = make()
    tplan = kernel_time_events(make, max(1, reps // 5))
    irr = hip.fock_to_irreps(sw["data"], *dev_args, t.orbital_template, block_data_offsets=sw["bdo"], plan=plan)
    tf = kernel_time_events(lambda: hip.fock_to_irreps(sw["data"], *dev_args, t.orbital_template,
                                                       block_data_offsets=sw["bdo"], plan=plan), reps)
    back = torch.zeros_like(sw["data"])
    ti = kernel_time_events(lambda: hip.irreps_to_fock(irr, back, *dev_args, t.orbital_template,
                                                       block_data_offsets=sw["bdo"], plan=plan), reps)
    rt = ((back - sw["data"]).abs().max() / sw["data"].abs().max()).item()
    tfp = kernel_time_events(lambda: hip.fock_to_irreps(sw["data"], *dev_args, t.orbital_template,
                                                        block_data_offsets=sw["bdo"]), reps)
    tip = kernel_time_events(lambda: hip.irreps_to_fock(irr, back, *dev_args, t.orbital_template,
                                                        block_data_offsets=sw["bdo"]), reps)
    nb = sw["n_blocks"]
    bpb = (sw["block_bytes"] + 4 * sw["T"] * nb) / nb
    return {"metric": "H-blocks/s", "fwd": nb / tf, "inv": nb / ti, "fwd_with_plan": nb / (tf + tplan),
            "inv_with_plan": nb / (ti + tplan), "fwd_pair_list": nb / tfp, "inv_pair_list": nb / tip,
            "plan_ms": tplan * 1e3, "blocks": nb, "T": sw["T"],
            "round_trip_rel_err": rt,
            "roofline": {"kernel": "transform_kernel<FOCK,ROWS> (block list)", "bound": "hbm",
                         "achieved": bpb * nb / tf / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                         "frac": bpb * nb / tf / PEAK_HBM, "bytes_per_block": bpb}}


def message_leg(cfg, dtype, steps, warmup, cpu=True):
    """fwd+bwd of the fused block on configuration ``cfg``: edges/s, the fused
    forward launch's MFMA roofline, and the CPU baseline."""
    import torch
    w = message_workload(dtype, cfg=cfg)
    t_step = time_steps(lambda: message_step(w, True), steps, warmup)
    t_fwd = time_steps(lambda: message_step(w, False), steps, warmup)
    t_launch = fused_forward_launch_time(w, reps=10)
    L, Mm, C, E = w["L"], w["M"], w["C"], w["E"]
    f_edge = fused_flops_per_edge(L, Mm, C, C) + (gated_flops_extra(L, C, C) if w["gate"] else 0)
    peak = PEAK_BF16 if dtype == "bf16" else PEAK_FP32
    gname = MESSAGE_CONFIGS[cfg][0]
    res = {"metric": "edges/s (fused block fwd+bwd)", "value": E / t_step, "ms_per_step": t_step * 1e3,
           "fwd_edges_per_s": E / t_fwd, "dtype": dtype,
           "config": {"workload": f"{cfg} fused message block fwd+bwd{' (gated)' if w['gate'] else ''}",
                      "graph": gname, "edges": E, "nodes": w["N"], "lmax": L, "mmax": Mm, "channels": C,
                      "gate": w["gate"], "rbf_cutoff_A": w["cutoff"]},
           "roofline": {"kernel": f"maloq_message_fwd: prep + gemm_kernel<{L},{Mm}> + fixup", "bound": "mfma",
                        "achieved": f_edge * E / t_launch / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                        "frac": f_edge * E / t_launch / peak, "flops_per_edge": f_edge,
                        "launch_ms": t_launch * 1e3}}
    del w
    torch.cuda.empty_cache()
    if cpu:
        res["cpu_baseline"] = cpu_message_baseline(budget_s=12.0, cfg=cfg)
    return res


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


TRAFFIC_JSON = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
# kernels that make up one launch of each measured entry point
TRAFFIC_GROUPS = {
    "message_fwd": r"maloq::msg::(prep_kernel|gemm_kernel|message_fixup_kernel)",
    "fock_to_irreps": r"maloq::bt::transform_kernel",
}
COPY_BYTES = 4 * 64 * 1024 * 1024        # the --only copy kernel: this many bytes read, as many written
PMC_GEMM = ("SQ_VALU_MFMA_BUSY_CYCLES", "GRBM_GUI_ACTIVE", "SQ_INSTS_MFMA", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
            "SQ_INSTS_VALU_MFMA_MOPS_F32", "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE")


def load_traffic(name):
    """HBM bytes per launch measured with rocprofv3 --pmc (profiles/traffic.json)."""
    try:
        return json.load(open(TRAFFIC_JSON)).get(name)
    except (OSError, ValueError):
        return None


def _pmc_medians(csv_path, counter):
    """Median per-dispatch value of `counter`, by kernel name, from a rocprofv3 CSV."""
    import csv
    import statistics
    vals = {}
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] == counter:
                vals.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return {k: statistics.median(v) for k, v in vals.items()}


def traffic_from(root, dtype):
    """Writes profiles/traffic.json from rocprofv3 --pmc runs under `root`:
    <root>/<piece>_<COUNTER>/run_counter_collection.csv for piece in copy, fwd,
    basis and COUNTER in FETCH_SIZE, WRITE_SIZE (KiB per dispatch).  Each
    counter is scaled by what it reads for the plain copy of known size."""
    import re
    out = {}
    scale = {}
    for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
        med = _pmc_medians(os.path.join(root, f"copy_{ctr}", "run_counter_collection.csv"), ctr)
        kib = max(med.values())
        scale[ctr] = COPY_BYTES / (kib * 1024.0)
    for name, piece in ((f"message_fwd_{dtype}", "fwd"), ("fock_to_irreps", "basis")):
        group = TRAFFIC_GROUPS[name.rsplit("_", 1)[0] if name.startswith("message") else name]
        tot = {}
        for ctr in ("FETCH_SIZE", "WRITE_SIZE"):
            med = _pmc_medians(os.path.join(root, f"{piece}_{ctr}", "run_counter_collection.csv"), ctr)
            tot[ctr] = sum(v for k, v in med.items() if re.search(group, k)) * 1024.0 * scale[ctr]
        out[name] = tot["FETCH_SIZE"] + tot["WRITE_SIZE"]
        out[name + "_read"] = tot["FETCH_SIZE"]
        out[name + "_write"] = tot["WRITE_SIZE"]
    out["copy_scale"] = scale
    try:
        prev = json.load(open(TRAFFIC_JSON))
    except (OSError, ValueError):
        prev = {}
    prev.update(out)
    with open(TRAFFIC_JSON, "w") as f:
        json.dump(prev, f, indent=1, sort_keys=True)
    print(json.dumps(out))
    return 0


COUNTER_PIECES = (("step_config2_fp32", "config 2, fp32, training step"),
                  ("step_config2_bf16", "config 2, bf16, training step"),
                  ("step_config4_bf16", "config 4 (lmax 6, gated), bf16, training step"),
                  ("step_config5_bf16", "config 5 (C 256), bf16, training step"),
                  ("edgewise_step_bf16", "Edgewise two convolutions, config 2, bf16, fwd+bwd"))
SIMDS = 1024  # 256 CUs x 4 SIMDs


def _kernel_label(name):
    """Short label of a message-block kernel from its demangled name, or None."""
    import re
    m = re.search(r"gemm_kernel<(\d+), (\d+), (true|false), (\d+), (\d+), maloq::msg::(\w+), (\d+), (\d+), "
                  r"(true|false), (\d+)>", name)
    if m:
        L, M, gate, nw, rt, tm, mode, kr, rad, minb = m.groups()
        modes = {"0": "FWD", "1": "BWD_DX", "2": "FWD_EDGE", "3": "BWD_EDGE"}
        return (f"gemm {modes[mode]} L{L} M{M}{' gated' if gate == 'true' else ''} {tm} "
                f"({32 * int(rt)}-edge tiles, {nw} waves{', radial grad' if rad == 'true' else ''})")
    for k in ("dw_tr_kernel", "dw_kernel", "dw_reduce_kernel", "prep_kernel", "radial_fwd", "radial_du",
              "radial_chain", "radial_dwo"):
        if k in name:
            return k + ("<BF16>" if "BF16" in name and k == "dw_kernel" else "<F32>" if k == "dw_kernel" else "")
    return None


def counters_from(root):
    """Writes profiles/gemm_counters.md from rocprofv3 --pmc runs under `root`:
    <root>/<piece>/run_counter_collection.csv for the COUNTER_PIECES (counters
    SQ_VALU_MFMA_BUSY_CYCLES, GRBM_GUI_ACTIVE, SQ_INSTS_MFMA,
    SQ_INSTS_VALU_MFMA_MOPS_BF16 / _F32, SQ_INSTS_LDS, SQ_LDS_BANK_CONFLICT,
    SQ_LDS_IDX_ACTIVE).  Per kernel the median dispatch: MFMA busy = busy
    cycles over (SIMDs x the dispatch's cycles, from GRBM_GUI_ACTIVE per XCD
    and its duration), MFMA TFLOP/s executed (MOPS x 512 over the duration),
    LDS bank-conflict cycles per LDS-active cycle."""
    import csv
    import statistics
    rows = ["| workload | kernel | dispatch µs | MFMA busy | MFMA TFLOP/s executed | MFMA instr. | LDS instr. | "
            "LDS bank conflicts / LDS active cycles |", "|---|---|---|---|---|---|---|---|"]
    for piece, what in COUNTER_PIECES:
        path = os.path.join(root, piece, "run_counter_collection.csv")
        if not os.path.exists(path):
            continue
        per = {}  # (label, dispatch) -> {counter: value, "dur": ns}
        with open(path) as f:
            for r in csv.DictReader(f):
                label = _kernel_label(r["Kernel_Name"])
                if label is None:
                    continue
                d = per.setdefault((label, r["Dispatch_Id"]), {})
                d[r["Counter_Name"]] = float(r["Counter_Value"])
                d["dur"] = float(r["End_Timestamp"]) - float(r["Start_Timestamp"])
        by = {}
        for (label, _), d in per.items():
            by.setdefault(label, []).append(d)
        for label in sorted(by):
            ds = by[label]
            med = lambda k: statistics.median(x.get(k, 0.0) for x in ds)
            dur = med("dur")
            grbm = med("GRBM_GUI_ACTIVE")
            xcds = max(1, round(grbm / (dur * 2.4))) if dur > 0 else 1  # GRBM summed over XCDs at ~2.4 GHz
            cycles = grbm / xcds
            busy = med("SQ_VALU_MFMA_BUSY_CYCLES") / (SIMDS * cycles) if cycles else 0.0
            mops = med("SQ_INSTS_VALU_MFMA_MOPS_BF16") + med("SQ_INSTS_VALU_MFMA_MOPS_F32")
            tflops = mops * 512 / (dur * 1e-9) / 1e12 if dur else 0.0
            conf = med("SQ_LDS_BANK_CONFLICT") / max(med("SQ_LDS_IDX_ACTIVE"), 1.0)
            rows.append(f"| {what} | {label} | {dur / 1e3:.1f} | {100 * busy:.1f} % | {tflops:.1f} | "
                        f"{med('SQ_INSTS_MFMA'):.3g} | {med('SQ_INSTS_LDS'):.3g} | {conf:.3f} |")
    out = os.path.join(os.path.dirname(TRAFFIC_JSON), "gemm_counters.md")
    with open(out, "w") as f:
        f.write("# MFMA and LDS counters of the message-block kernels (rocprofv3 --pmc, median dispatch)\n\n")
        f.write("Commands (GPU box, repo root, one counter pass per workload):\n\n")
        for piece, what in COUNTER_PIECES:
            only = "edgewise-step" if piece.startswith("edgewise") else "step"
            dt = piece.rsplit("_", 1)[1]
            cfg = "" if only != "step" else f" --cfg {piece.split('_')[1]}"
            f.write(f"    timeout -s KILL 90 rocprofv3 --pmc {' '.join(PMC_GEMM)} --output-format csv "
                    f"-d <root>/{piece} -o run -- python bench.py --only {only} --dtype {dt}{cfg} --reps 2\n")
        f.write(f"    python bench.py --counters-from <root>\n\n")
        f.write("MFMA busy: SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x the dispatch's cycles); the cycles are "
                "GRBM_GUI_ACTIVE per XCD (the counter is summed over the XCDs).  MFMA TFLOP/s executed: "
                "(SQ_INSTS_VALU_MFMA_MOPS_BF16 + _F32) x 512 / dispatch time (peaks: bf16 2500, fp32 157.3).  "
                "Durations are those of the counter run (kernels serialised).\n\n")
        f.write("\n".join(rows) + "\n")
    print(open(out).read())
    return 0


def embed_workload(seed=0):
    """Config-2 edge-degree embedding (EdgeDegreeEmbedding, node mode): radial
    rows [E, (L+1) C] fp32, Euler angles, the dst plan, x [N, d, C] fp32."""
    import numpy as np
    import torch
    from maloq_amd import message as M
    from maloq_amd import synth
    from maloq_amd.wigner import extract_euler_angles

    dev = torch.device("cuda:0")
    g = synth.config2_graph()
    L, C = 4, 128
    gen = torch.Generator().manual_seed(seed)
    ei = torch.from_numpy(np.stack([g.src, g.dst])).to(dev)
    plan = M.MessagePlan(ei, g.num_nodes)
    vec = torch.from_numpy(g.edge_distance_vec()).float().to(dev)
    eul = extract_euler_angles(vec, seed=1234)
    u = torch.randn(g.num_edges, (L + 1) * C, generator=gen).to(dev)
    x = torch.zeros(g.num_nodes, (L + 1) ** 2, C, device=dev)
    E, N, d = g.num_edges, g.num_nodes, (L + 1) ** 2
    nbytes = E * (L + 1) * C * 4 + E * 12 + E * 8 + (N + 1) * 8 + 2 * N * d * C * 4
    return dict(ei=ei, plan=plan, eul=eul, u=u, x=x, L=L, C=C, E=E, N=N, bytes=nbytes, vec=vec)


def embed_call(ew):
    import torch
    from maloq_amd.embedding import edge_degree_embed
    with torch.no_grad():
        edge_degree_embed(ew["x"], ew["u"], ew["ei"], None, ew["L"], 5.0, "node", eulers=ew["eul"], plan=ew["plan"])


def cpu_embed_baseline(ew):
    """The oracle restatement of EdgeDegreeEmbedding.forward (fp32 torch on the
    host cores: pad, einsum to_m, bmm(wigner_inv), index_add_) on the whole
    config-2 graph, median of 3; the dense wigner_inv is built once beforehand
    (not timed), as the reference receives it."""
    import torch
    from oracle import embedding as oemb
    from oracle import rotation as orot
    from oracle.so3 import CoefficientMapping
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    L = ew["L"]
    e = ew["eul"].cpu()
    winv = orot.eulers_to_wigner((e[:, 0], e[:, 1], e[:, 2]), 0, L, orot.load_jd(torch.float32)).transpose(1, 2)
    winv = winv.contiguous()
    mapping = CoefficientMapping(L, 2)
    mask = CoefficientMapping(L, L).coefficient_idx(L, 2)
    u, ei, x = ew["u"].cpu(), ew["ei"].cpu(), ew["x"].cpu().zero_()
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        oemb.edge_degree_embedding(x, u, ei, winv, mapping, mask, 5.0, "node")
        times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    return {"value": ew["E"] / t, "unit": "edges/s", "cores": cores, "kind": "port",
            "sample": f"config 2, whole graph ({ew['E']} edges), fp32 torch CPU, median of 3"}


def edgewise_flops_per_edge(L, M, c, h):
    """Algorithmic FLOPs per edge of the two-convolution Edgewise forward:
    rotation of the 2c-channel message, gated SO(2) 2c -> h (plus the L h gate
    rows of m = 0), SO(2) h -> c, inverse rotation, segment sum."""
    rot = sum(min(2 * l + 1, 2 * M + 1) * (2 * l + 1) for l in range(L + 1))
    m_side = sum(4 * (L - m + 1) ** 2 for m in range(1, M + 1))
    mac1 = (L + 1) * 2 * c * (2 * L + 1) * h + m_side * 2 * c * h
    mac2 = (L + 1) ** 2 * h * c + m_side * h * c
    return 2 * (rot * 2 * c + mac1 + mac2 + rot * c) + (L + 1) ** 2 * c


def edgewise_workload(seed=0):
    """Config-2 graph through Edgewise (message_type "source-target"): x [N, 25,
    128] bf16, conv1 256 -> 128 gated with radial scales, conv2 128 -> 128."""
    import torch
    from maloq_amd import message as M
    w = message_workload("bf16", seed)
    dev, L, Mm, C = w["x"].device, w["L"], w["M"], w["C"]
    H = C
    gen = torch.Generator().manual_seed(seed + 1)

    def conv(c_in, c_out, extra):
        k0 = (L + 1) * c_in
        w0 = (torch.randn((L + 1) * c_out + extra, k0, generator=gen) / math.sqrt(k0)).to(dev)
        b0 = (torch.randn((L + 1) * c_out + extra, generator=gen) * 0.1).to(dev)
        wm = [(torch.randn(2 * (L - m + 1) * c_out, (L - m + 1) * c_in, generator=gen)
               / math.sqrt((L - m + 1) * c_in)).to(dev) for m in range(1, Mm + 1)]
        return w0, b0, wm
    c1, c2 = conv(2 * C, H, L * H), conv(H, C, 0)
    wp1 = M.pack_weights(c1[0], c1[2], L, Mm, True, 2 * C, H, torch.bfloat16, 0)
    wp2 = M.pack_weights(c2[0], c2[2], L, Mm, False, H, C, torch.bfloat16, 0)
    with torch.no_grad():
        from maloq_amd.wigner import extract_euler_angles
        eul = extract_euler_angles(w["vec"], seed=1234)
        rad = (torch.rand(w["E"], M.rad_width(L, Mm, 2 * C), generator=gen) + 0.5).to(dev, torch.bfloat16)
    return dict(x=w["x"].detach(), plan=w["plan"], eul=eul, rad=rad, c1=c1, c2=c2, wp1=wp1, wp2=wp2,
                L=L, M=Mm, C=C, H=H, E=w["E"])


def edgewise_call(ew):
    import torch
    from maloq_amd import message as M
    with torch.no_grad():
        return M.edgewise_forward(ew["x"], ew["plan"], ew["eul"], ew["rad"], ew["c1"], ew["c2"], ew["L"], ew["M"],
                                  wpack1=ew["wp1"], wpack2=ew["wp2"])


def edgewise_step(ew):
    """Forward + backward of the two-convolution block (gradients of x, the
    radial scales and both convolutions' weights and biases), from cleared
    gradients."""
    from maloq_amd import message as M
    if "leaves" not in ew:
        c1 = tuple(t.detach().clone().requires_grad_() for t in ew["c1"][:2]) + \
            ([w.detach().clone().requires_grad_() for w in ew["c1"][2]],)
        c2 = tuple(t.detach().clone().requires_grad_() for t in ew["c2"][:2]) + \
            ([w.detach().clone().requires_grad_() for w in ew["c2"][2]],)
        ew["leaves"] = (ew["x"].detach().clone().requires_grad_(), ew["rad"].detach().clone().requires_grad_(), c1, c2)
        ew["gout"] = torch_randn_like_nodes(ew)
    x, rad, c1, c2 = ew["leaves"]
    for t in [x, rad, c1[0], c1[1], *c1[2], c2[0], c2[1], *c2[2]]:
        t.grad = None
    out = M.edgewise_block(x, ew["plan"], ew["eul"], rad, c1, c2, ew["L"], ew["M"])
    out.backward(ew["gout"])


REF_LAYERS = 4


def reference_backbone_workload(dtype_name, seed=0, lmax=4, layers=None):
    """The reference's layer loop (helm/esen_osh.py:438-463) on the config-2
    graph: REF_LAYERS Edgewise modules at its model shape (lmax = mmax = 4,
    sphere and hidden channels 128, radial [384, 128, 128], training_workflow.py:
    508-511, run_QM7.py:66-67), called with its signature: the dense wigner and
    wigner_inv [E, 25, 25] and one edge_index tensor, no plan (the modules find
    the graph's plan in the cache)."""
    import numpy as np
    import torch
    from maloq_amd.edgewise import Edgewise
    from maloq_amd.so3 import CoefficientMapping
    from maloq_amd.wigner import extract_euler_angles, wigner_from_eulers
    dev = torch.device("cuda:0")
    dt = {"bf16": torch.bfloat16, "fp32": torch.float32}[dtype_name]
    g = _graph("config2_graph")
    L = Mm = lmax
    C = H = 128
    torch.manual_seed(seed)
    mods = [Edgewise(C, H, L, Mm, [384, 128, 128], CoefficientMapping(L, Mm), None, 6.0, "source-target").to(dev)
            for _ in range(REF_LAYERS if layers is None else layers)]
    gen = torch.Generator().manual_seed(seed)
    ei = torch.from_numpy(np.stack([g.src, g.dst])).to(dev)
    vec = torch.from_numpy(g.edge_distance_vec()).float().to(dev)
    with torch.no_grad():
        wig = wigner_from_eulers(extract_euler_angles(vec, seed=3), None, L)
        wig_inv = wig.transpose(1, 2).contiguous()
    x = torch.randn(g.num_nodes, (L + 1) ** 2, C, generator=gen).to(dev, dt).requires_grad_()
    x_edge = torch.randn(g.num_edges, 384, generator=gen).to(dev).requires_grad_()
    return dict(mods=mods, ei=ei, wig=wig, wig_inv=wig_inv, x=x, x_edge=x_edge, L=L, M=Mm, C=C, H=H,
                E=g.num_edges, N=g.num_nodes, dt=dt)


def reference_backbone_pass(rw, backward=True, cached=True):
    """The layer loop: x <- x + Edgewise_i(x), then the gradient of a fixed
    linear loss wrt x, x_edge and every module parameter.  cached=False drops
    the plan cache before each layer (the plan built per call, as without it)."""
    import torch
    from maloq_amd import message as M
    x = rw["x"]
    for t in [rw["x"], rw["x_edge"], *[p for m in rw["mods"] for p in m.parameters()]]:
        t.grad = None
    with torch.set_grad_enabled(backward):
        h = x
        for mod in rw["mods"]:
            if not cached:
                M.clear_plan_cache()
            h = h + mod(h, None, rw["x_edge"], rw["ei"], rw["wig"], rw["wig_inv"], "node").to(h.dtype)
        if backward:
            h.float().sum().backward()
    return h


def reference_backbone_leg(dtype_name, steps=5, warmup=2, cpu=True, lmax=4, layers=None):
    import torch
    from maloq_amd import message as M
    rw = reference_backbone_workload(dtype_name, lmax=lmax, layers=layers)
    M.clear_plan_cache()
    built0 = M._PLANS.built
    reference_backbone_pass(rw, True)
    plans_per_pass = M._PLANS.built - built0
    t_step = time_steps(lambda: reference_backbone_pass(rw, True), steps, warmup)
    t_fwd = time_steps(lambda: reference_backbone_pass(rw, False), steps, warmup)
    t_fwd_nc = time_steps(lambda: reference_backbone_pass(rw, False, cached=False), steps, warmup)
    E, n = rw["E"], len(rw["mods"])
    fl = edgewise_flops_per_edge(rw["L"], rw["M"], rw["C"], rw["H"]) * E * n
    peak = PEAK_BF16 if dtype_name == "bf16" else PEAK_FP32
    out = {"metric": "edges/s per layer", "fwd_bwd": E * n / t_step, "fwd": E * n / t_fwd,
           "fwd_without_plan_cache": E * n / t_fwd_nc, "ms_per_pass_fwd_bwd": t_step * 1e3,
           "ms_per_pass_fwd": t_fwd * 1e3, "ms_per_pass_fwd_without_plan_cache": t_fwd_nc * 1e3,
           "plans_built_per_pass": plans_per_pass, "layers": n, "dtype": dtype_name,
           "config": f"config-2 graph (36 804 edges), Edgewise x{n} at the reference's model shape: "
                     f"lmax = mmax = {rw['L']}, C = H = 128, radial [384, 128, 128], dense wigner / wigner_inv, "
                     "no plan= (reference call)",
           "roofline": {"scope": "whole forward pass (radial MLPs, Wigner-row gathers, prep, both GEMMs, fixups)",
                        "bound": "mfma", "achieved": fl / t_fwd / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                        "frac": fl / t_fwd / peak, "flops_per_pass": fl}}
    if cpu:
        out["cpu_baseline"] = cpu_reference_backbone_baseline(rw)
    del rw
    torch.cuda.empty_cache()
    return out


def cpu_reference_backbone_baseline(rw, budget_s=10.0):
    """The oracle's two-convolution Edgewise (oracle.message.message_block with
    conv2, concat source-target, fp32 torch on the host cores), one layer forward
    + backward, on the in-edges of the graph's first nodes, against the module's
    own weights (radial scales precomputed: the layer's SO(2) work)."""
    import numpy as np
    import torch
    from oracle import message as omsg
    from oracle import rotation as orot
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    mod = rw["mods"][0]
    L, Mm, C, H = rw["L"], rw["M"], rw["C"], rw["H"]
    g = _graph("config2_graph")
    sel = torch.from_numpy(g.mol[g.dst] == 0)  # the first molecule's in-edges
    ei = torch.from_numpy(np.stack([g.src, g.dst]))[:, sel]
    vec = torch.from_numpy(g.edge_distance_vec()).float()[sel]
    eul = extract_euler_angles(vec.to("cuda:0"), seed=3).cpu()
    cpu = lambda t: t.detach().float().cpu()
    conv = lambda c, co: {"w0": cpu(c.fc_m0.weight).requires_grad_(), "b0": cpu(c.fc_m0.bias).requires_grad_(),
                          "wm": [cpu(m.fc.weight).requires_grad_() for m in c.so2_m_conv], "c_out": co}
    c1, c2 = conv(mod.so2_conv_1, H), conv(mod.so2_conv_2, C)
    x = torch.randn(g.num_nodes, (L + 1) ** 2, C).requires_grad_()
    rad = (torch.rand(ei.shape[1], M.rad_width(L, Mm, 2 * C)) + 0.5).requires_grad_()
    jd = orot.load_jd()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t0 = time.perf_counter()
        out = omsg.message_block(x, ei, (eul[:, 0], eul[:, 1], eul[:, 2]), jd, L, Mm, c1, rad=rad, conv2=c2,
                                 gate=True, concat="source-target")
        out.sum().backward()
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    return {"value": ei.shape[1] / t, "unit": "edges/s per layer", "cores": cores, "kind": "port",
            "sample": f"one layer fwd+bwd on the {ei.shape[1]} in-edges of the first molecule (config 2), fp32 "
                      f"torch, median of {len(times)}"}


def torch_randn_like_nodes(ew):
    import torch
    gen = torch.Generator().manual_seed(7)
    return torch.randn(ew["x"].shape, generator=gen).to(ew["x"].device)


def library_gemm_ceiling(dtypes=("bf16", "fp32"), reps=20):
    """The SO(2) per-m GEMMs of each message configuration as plain library
    GEMMs (torch.matmul -> hipBLASLt), no rotation or scatter: Y_m [E, k] x
    W_m [k, k] with k = (L+1) C for m = 0 and 2 (L-m+1) C for m > 0 (the +-m
    complex mix as one real GEMM) -- the same FLOPs as the fused kernel's SO(2)
    part.  The achievable rate of the library on these shapes."""
    import torch
    dev = torch.device("cuda:0")
    out = {}
    for cfg, (gname, L, M, C, gate, _) in MESSAGE_CONFIGS.items():
        if cfg == "config1":   # the host-overhead case only
            continue
        E = _graph(gname).src.shape[0]
        for dtn in dtypes:
            dt = torch.bfloat16 if dtn == "bf16" else torch.float32
            gen = torch.Generator(device="cpu").manual_seed(0)
            parts, tot_f, tot_t = {}, 0.0, 0.0
            for m in range(M + 1):
                k = (L - m + 1) * C * (1 if m == 0 else 2)
                kn = k + (L * C if (m == 0 and gate) else 0)   # gated: the gate outputs ride on m = 0
                y = torch.randn(E, k, generator=gen).to(dev, dt)
                w = torch.randn(k, kn, generator=gen).to(dev, dt)
                tm = kernel_time_events(lambda y=y, w=w: torch.matmul(y, w), reps)
                fl = 2.0 * E * k * kn
                parts[f"m{m}"] = {"shape": [E, k, kn], "us": tm * 1e6, "tflops": fl / tm / 1e12}
                tot_f += fl
                tot_t += tm
                del y, w
            peak = PEAK_BF16 if dtn == "bf16" else PEAK_FP32
            out[f"{cfg}_{dtn}"] = {"us": tot_t * 1e6, "tflops": tot_f / tot_t / 1e12,
                                   "frac_of_peak": tot_f / tot_t / peak, "per_m": parts}
    return out


def profile_only(args):
    """Runs one piece of the path --reps times (for rocprofv3 passes)."""
    import torch
    if args.only == "copy":
        # plain copy of a known size: calibrates FETCH_SIZE / WRITE_SIZE
        a = torch.ones(64 * 1024 * 1024, device="cuda")
        b = torch.empty_like(a)
        for _ in range(args.reps):
            b.copy_(a)
    elif args.only == "host":
        # wall time per training step through the module path and through the
        # registered operators: config 1 (132 edges) is bound by the host's
        # enqueue, config 2 by the GPU
        res = {}
        for cfg in ("config1", "config2"):
            w = message_workload(args.dtype, cfg=cfg)
            for name, use_ops in (("module", False), ("ops", True)):
                t = time_steps(lambda: message_step(w, ops=use_ops), max(args.reps, 20), 5)
                res[f"{cfg}_{name}_us_per_step"] = t * 1e6
        print(json.dumps(res), flush=True)
    elif args.only == "hbm":
        # the practical HBM ceiling of the box: torch's device copy (read +
        # write), fill (write) and sum (read) over one fp32 [E, d, C] array of
        # config 2 (471 MB), event-timed
        n = 36804 * 25 * 128
        a = torch.ones(n, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
            b.fill_(1.0)
            a.sum()
        torch.cuda.synchronize()
        nb = 4 * n
        tc = kernel_time_events(lambda: b.copy_(a), args.reps)
        tf = kernel_time_events(lambda: b.fill_(2.0), args.reps)
        ts = kernel_time_events(lambda: a.sum(), args.reps)
        print(json.dumps({"bytes_per_array": nb, "copy_TBps": 2 * nb / tc / 1e12, "fill_TBps": nb / tf / 1e12,
                          "sum_TBps": nb / ts / 1e12, "copy_us": tc * 1e6, "peak_TBps": 8.0}), flush=True)
    elif args.only == "embed":
        ew = embed_workload()
        for _ in range(args.reps):
            embed_call(ew)
    elif args.only == "edgewise":
        ew = edgewise_workload()
        for _ in range(args.reps):
            edgewise_call(ew)
    elif args.only == "edgewise-step":
        ew = edgewise_workload()
        for _ in range(args.reps):
            edgewise_step(ew)
    elif args.only == "rotate":
        rotation_leg(cpu=False)
    elif args.only == "ceiling":
        print(json.dumps(library_gemm_ceiling()), flush=True)
    elif args.only == "basis5":
        sw = sparse_basis_workload()
        sparse_basis_leg(sw, reps=args.reps)
    elif args.only == "ref-backbone":
        rw = reference_backbone_workload(args.dtype)
        for _ in range(args.reps):
            reference_backbone_pass(rw, True)
    elif args.only == "ref-layer6":
        # one layer at lmax = mmax = 6; prints its bench leg (no CPU baseline)
        print(json.dumps(reference_backbone_leg(args.dtype, steps=args.reps, warmup=1, cpu=False, lmax=6,
                                                layers=1)), flush=True)
    elif args.only == "fock-head":
        print(json.dumps(fock_head_leg(reps=max(args.reps, 5))), flush=True)
    elif args.only == "graph-step":
        print(json.dumps({c: graph_step_leg(c, args.dtype, reps=max(args.reps, 10)) for c in ("config1", "config2")}),
              flush=True)
    elif args.only == "basis-tzvpd":
        print(json.dumps(wide_basis_leg(reps=args.reps, cpu=False)), flush=True)
    elif args.only in ("fwd", "step"):
        w = message_workload(args.dtype, cfg=args.cfg)
        if args.only == "fwd":
            # the bench times the forward after its training steps: warm the GPU
            # the same way, so that a profile of this mode matches the headline
            for _ in range(20):
                message_step(w, True)
            t = fused_forward_launch_time(w, reps=args.reps)
            print(json.dumps({"fused_forward_launch_us": t * 1e6, "cfg": args.cfg, "dtype": args.dtype,
                              "reps": args.reps}), flush=True)
        else:
            for _ in range(args.reps):
                message_step(w, True)
    else:
        # forward transform only, so its counters are not mixed with the inverse
        import numpy as np
        bw = basis_workload()
        hip, t = bw["hip"], bw["tables"]
        dev = bw["data"].device
        dev_args = tuple(torch.as_tensor(np.asarray(a, np.int32), device=dev)
                         for a in (bw["off"], bw["Z"], bw["rows"], bw["cols"]))
        plan = hip.make_plan(bw["data"], *dev_args, t.orbital_template, block_data_offsets=bw["bdo"])
        for _ in range(args.reps):
            hip.fock_to_irreps(bw["data"], *dev_args, t.orbital_template, block_data_offsets=bw["bdo"], plan=plan)
    torch.cuda.synchronize()
    print(f"[bench] --only {args.only}: {args.reps} reps done", file=sys.stderr, flush=True)
    return 0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--dtype", default="fp32", choices=["bf16", "fp32"],
                    help="precision of the headline (the reference computes in fp32)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-extras", action="store_true", help="headline only")
    ap.add_argument("--only", choices=["fwd", "step", "basis", "copy", "hbm", "host", "graph-step", "fock-head", "embed", "edgewise", "edgewise-step",
                                       "rotate", "basis5", "basis-tzvpd", "ref-backbone", "ref-layer6", "ceiling"],
                    help="profiling mode: run one piece a few times and exit (no JSON line)")
    ap.add_argument("--cfg", default="config2", choices=sorted(MESSAGE_CONFIGS),
                    help="message-block configuration of --only fwd / step")
    ap.add_argument("--reps", type=int, default=5, help="launches in --only mode")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="write profiles/traffic.json from rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE runs in DIR")
    ap.add_argument("--counters-from", metavar="DIR",
                    help="write profiles/gemm_counters.md from rocprofv3 --pmc MFMA/LDS counter runs in DIR")
    args = ap.parse_args(argv)
    if args.traffic_from:
        return traffic_from(args.traffic_from, args.dtype)
    if args.counters_from:
        return counters_from(args.counters_from)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the hot path runs on a single MI355X; multi-GPU sharding is design-only)", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    if args.only:
        return profile_only(args)
    print(f"[bench] workload: config 2 fused message block ({args.dtype}) ...", file=sys.stderr, flush=True)
    w = message_workload(args.dtype)
    t_step = time_steps(lambda: message_step(w, True), args.steps, args.warmup)
    E = w["E"]
    print(f"[bench] fwd+bwd {t_step * 1e3:.3f} ms/step, {E / t_step:.4g} edges/s", file=sys.stderr, flush=True)
    t_fwd_launch = fused_forward_launch_time(w)
    f_edge = fused_flops_per_edge(w["L"], w["M"], w["C"], w["C"])
    peak = PEAK_BF16 if args.dtype == "bf16" else PEAK_FP32
    achieved = f_edge * E / t_fwd_launch
    t_fwd_step = time_steps(lambda: message_step(w, False), args.steps, args.warmup)
    result = {
        "metric": "edges/sec fused rotate+SO2 (lmax=4,C=128); H-blocks/sec basis transform; %roofline",
        "value": E / t_step,
        "unit": "edges/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": t_step * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.dtype,
        "data": "synthetic (seeded config-2 geometry, random-init weights)",
        "config": {"workload": "config2 fused message block fwd+bwd: Euler/Wigner-D, radial MLP, "
                               "rotate->SO(2)->inverse rotate->segment sum, input/radial/weight grads",
                   "molecules": 32, "atoms_per_molecule": 40, "edges": E, "nodes": w["N"],
                   "lmax": w["L"], "mmax": w["M"], "channels": w["C"], "rbf": 8, "cutoff_A": 6.0},
        "roofline": {"kernel": "maloq_message_forward: prep + gemm_kernel<4,2> + fixup", "bound": "mfma",
                     "achieved": achieved / 1e12, "peak": peak / 1e12, "unit": "TFLOP/s",
                     "frac": achieved / peak, "traffic": load_traffic(f"message_fwd_{args.dtype}"),
                     "flops_per_edge": f_edge, "launch_ms": t_fwd_launch * 1e3},
        "fwd_edges_per_s": E / t_fwd_step,
    }
    del w
    torch.cuda.empty_cache()
    other = "bf16" if args.dtype == "fp32" else "fp32"
    if not args.no_extras:
        # the same configuration in the other precision (the reference computes in fp32)
        print(f"[bench] config 2 in {other} ...", file=sys.stderr, flush=True)
        result[f"config2_{other}"] = message_leg("config2", other, max(5, args.steps // 2), 3, cpu=False)
        print("[bench] config 1 rotation ...", file=sys.stderr, flush=True)
        result["config1_rotation"] = rotation_leg(cpu=not args.no_cpu)
        print("[bench] training step replayed from a HIP graph (config 1, config 2) ...", file=sys.stderr, flush=True)
        result["hip_graph_step"] = {c: graph_step_leg(c, "fp32", reps=50 if c == "config1" else 10)
                                    for c in ("config1", "config2")}
        for cfg in ("config4", "config5"):
            print(f"[bench] {cfg} fused block (bf16) ...", file=sys.stderr, flush=True)
            result[cfg] = message_leg(cfg, "bf16", max(5, args.steps // 2), 3, cpu=not args.no_cpu)
        print("[bench] basis transform (config 3) ...", file=sys.stderr, flush=True)
        bw = basis_workload()
        tf, ti, rt, tplan, tfp, tip = basis_timing(bw)
        bpb = (bw["block_bytes"] + 4 * bw["T"] * bw["n_blocks"]) / bw["n_blocks"]
        result["basis_transform"] = {
            "metric": "H-blocks/s", "fwd": bw["n_blocks"] / tf, "inv": bw["n_blocks"] / ti,
            "fwd_with_plan": bw["n_blocks"] / (tf + tplan), "inv_with_plan": bw["n_blocks"] / (ti + tplan),
            "fwd_pair_list": bw["n_blocks"] / tfp, "inv_pair_list": bw["n_blocks"] / tip,
            "blocks": bw["n_blocks"], "round_trip_rel_err": rt, "plan_ms": tplan * 1e3,
            "roofline": {"bound": "hbm", "achieved": bpb * bw["n_blocks"] / tf / 1e9, "peak": PEAK_HBM / 1e9,
                         "unit": "GB/s", "frac": bpb * bw["n_blocks"] / tf / PEAK_HBM,
                         "bytes_per_block": bpb, "traffic": load_traffic("fock_to_irreps")},
        }
        print("[bench] basis transform (config 5, block list) ...", file=sys.stderr, flush=True)
        sw = sparse_basis_workload()
        result["config5_basis_transform"] = sparse_basis_leg(sw)
        if not args.no_cpu:
            result["config5_basis_transform"]["cpu_baseline"] = cpu_sparse_basis_baseline(sw)
        del sw
        print("[bench] basis transform (config 3 molecules, def2-TZVPD template) ...", file=sys.stderr, flush=True)
        result["def2_tzvpd_basis_transform"] = wide_basis_leg(cpu=not args.no_cpu)
        print("[bench] Fock_Irreps_Head and eval formats (config 3) ...", file=sys.stderr, flush=True)
        result["fock_irreps_head"] = fock_head_leg()
        print("[bench] edge-degree embedding (config 2) ...", file=sys.stderr, flush=True)
        ew = embed_workload()
        s = torch.cuda.current_stream()
        embed_call(ew)
        s.synchronize()
        a_ev, b_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a_ev.record(s)
        for _ in range(20):
            embed_call(ew)
        b_ev.record(s)
        b_ev.synchronize()
        te = a_ev.elapsed_time(b_ev) / 1e3 / 20
        result["edge_degree_embedding"] = {
            "metric": "edges/s", "value": ew["E"] / te, "us_per_call": te * 1e6,
            "config": "config 2 node mode, fp32 radial rows, D from Euler angles",
            "roofline": {"kernel": "edge_degree_node_kernel<4>", "bound": "hbm",
                         "achieved": ew["bytes"] / te / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                         "frac": ew["bytes"] / te / PEAK_HBM, "bytes_per_call": ew["bytes"]},
        }
        print("[bench] Edgewise two convolutions (config 2) ...", file=sys.stderr, flush=True)
        gw = edgewise_workload()
        edgewise_call(gw)
        tg = kernel_time_events(lambda: edgewise_call(gw), 20)
        fl = edgewise_flops_per_edge(gw["L"], gw["M"], gw["C"], gw["H"]) * gw["E"]
        ts = time_steps(lambda: edgewise_step(gw), 10, 3)
        result["edgewise_two_conv"] = {
            "metric": "edges/s", "value": gw["E"] / tg, "us_per_call": tg * 1e6,
            "fwd_bwd_edges_per_s": gw["E"] / ts, "fwd_bwd_ms": ts * 1e3,
            "config": "config 2 graph, cat(x[src], x[dst]) 256 -> gated 128 -> 128 channels, bf16; value: forward, "
                      "fwd_bwd: forward + all gradients",
            "roofline": {"scope": "whole call (prep, two GEMMs, fixup)", "bound": "mfma",
                         "achieved": fl / tg / 1e12, "peak": PEAK_BF16 / 1e12, "unit": "TFLOP/s",
                         "frac": fl / tg / PEAK_BF16, "flops_per_call": fl},
        }
        del gw
        for dtn in ("fp32", "bf16"):
            print(f"[bench] reference layer loop (Edgewise x{REF_LAYERS}, lmax = mmax = 4, {dtn}) ...",
                  file=sys.stderr, flush=True)
            result[f"reference_backbone_{dtn}"] = reference_backbone_leg(dtn, cpu=(dtn == "fp32" and not args.no_cpu))
        for dtn in ("fp32", "bf16"):
            print(f"[bench] reference layer at lmax = mmax = 6 (Edgewise x1, {dtn}) ...", file=sys.stderr, flush=True)
            result[f"reference_layer_l6_{dtn}"] = reference_backbone_leg(
                dtn, steps=3, warmup=1, cpu=(dtn == "fp32" and not args.no_cpu), lmax=6, layers=1)
        print("[bench] library GEMM ceiling of the SO(2) shapes ...", file=sys.stderr, flush=True)
        result["library_gemm_ceiling"] = library_gemm_ceiling(("bf16",))
    if not args.no_cpu:
        print("[bench] CPU baseline ...", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_message_baseline()
        if not args.no_extras:
            result["basis_transform"]["cpu_baseline"] = cpu_basis_baseline(bw)
            result["edge_degree_embedding"]["cpu_baseline"] = cpu_embed_baseline(ew)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
