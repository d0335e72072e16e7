#!/usr/bin/env python3
"""Benchmark of MALOQ's equivariant message-passing hot path on one MI355X.

Headline workload: the reference benchmark's config 2 (32 molecules x 40
atoms, ~30k directed edges, lmax 4, mmax 2, 128 channels, 8 Gaussian RBFs).
A step is one fused message block, forward and backward, with inputs already
resident in HBM: per-edge Euler angles + Wigner-D, the radial MLP (fused HIP), the
fused rotate -> SO(2) -> inverse-rotate -> segment-sum kernel, and its input,
radial and weight gradients.  `value` is edges per second.

The JSON line also carries the roofline of the dominant kernel (the fused
forward launch, MFMA-bound), the CPU baseline (the build's own CPU
restatement of the reference's PyTorch path, timed on a bounded sample) and
the basis-transform throughput (config 3, H-blocks/s) with its HBM roofline.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--dtype bf16|fp32]
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


def gaussian_rbf(dist, start, stop, num):
    import torch
    offset = torch.linspace(start, stop, num, device=dist.device)
    coeff = -0.5 / (offset[1] - offset[0]).item() ** 2
    return torch.exp(coeff * (dist.view(-1, 1) - offset.view(1, -1)) ** 2)


def message_workload(dtype_name, seed=0):
    """Tensors of config 2 on cuda:0."""
    import numpy as np
    import torch
    from maloq_amd import message as M
    from maloq_amd import synth

    dev = torch.device("cuda:0")
    dt = {"bf16": torch.bfloat16, "fp32": torch.float32}[dtype_name]
    g = synth.config2_graph()
    L, Mm, C = 4, 2, 128
    gen = torch.Generator().manual_seed(seed)
    N, E = g.num_nodes, g.num_edges
    plan = M.MessagePlan(torch.from_numpy(np.stack([g.src, g.dst])).to(dev), N)
    vec = plan.sort_edges(torch.from_numpy(g.edge_distance_vec()).float().to(dev))
    dist = vec.norm(dim=1)
    x = torch.randn(N, (L + 1) ** 2, C, generator=gen).to(device=dev, dtype=dt).requires_grad_()
    k0 = (L + 1) * C
    w0 = (torch.randn((L + 1) * C, k0, generator=gen) / math.sqrt(k0)).to(dev).requires_grad_()
    b0 = torch.zeros((L + 1) * C, device=dev, requires_grad=True)
    wm = []
    for m in range(1, Mm + 1):
        k = (L - m + 1) * C
        wm.append((torch.randn(2 * (L - m + 1) * C, k, generator=gen) / math.sqrt(k)).to(dev).requires_grad_())
    torch.manual_seed(seed)
    radial = make_radial(8, 64, M.rad_width(L, Mm, C), dev)
    gout = torch.randn(N, (L + 1) ** 2, C, generator=gen).to(dev)
    return dict(graph=g, plan=plan, vec=vec, dist=dist, x=x, w0=w0, b0=b0, wm=wm, radial=radial,
                gout=gout, L=L, M=Mm, C=C, dt=dt, N=N, E=E)


def message_step(w, backward=True):
    from maloq_amd import message as M
    from maloq_amd.wigner import extract_euler_angles
    eul = extract_euler_angles(w["vec"], seed=1234)
    rad = w["radial"](gaussian_rbf(w["dist"], 0.0, 6.0, 8), out_dtype=w["dt"])
    out = M.message_block(w["x"], w["plan"], eul, rad, w["w0"], w["b0"], w["wm"], w["L"], w["M"])
    if backward:
        # a training step starts from cleared gradients (zero_grad(set_to_none=True))
        for t in [w["x"], w["w0"], w["b0"], *w["wm"], *w["radial"].parameters()]:
            t.grad = None
        out.backward(w["gout"])
    return out


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
        rad = w["radial"](gaussian_rbf(w["dist"], 0.0, 6.0, 8), out_dtype=w["dt"])
        x = w["x"].detach()
        wpack = M.pack_weights(w["w0"], w["wm"], w["L"], w["M"], False, w["C"], w["C"], w["dt"], 0)
        f = lambda: M.message_forward(x, w["plan"], eul, rad, w["w0"], w["b0"], w["wm"], w["L"], w["M"],
                                      wpack=wpack)
        return kernel_time_events(f, reps)


# ---------------------------------------------------------- basis transform
CFG3_BASIS = {1: [0, 0, 1], 6: [0, 0, 0, 1, 1, 2], 7: [0, 0, 0, 1, 1, 2], 8: [0, 0, 0, 1, 1, 2]}


def basis_workload():
    """Config 3 as one block list (all on-site + off-site < 8 A blocks of 64
    molecules), so the whole batch is one launch."""
    import numpy as np
    import torch
    from maloq_amd import synth
    from maloq_amd import tensor_decomp as ptd
    from maloq_amd.basis_transform import HipE3TensorDecomp

    dev = torch.device("cuda:0")
    t = ptd.BasisTables(CFG3_BASIS)
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
    return fwd, inv, rt, plan_s


# ---------------------------------------------------------------- CPU legs
def cpu_message_baseline(budget_s=15.0):
    """The build's CPU restatement of the reference path (bmm(wigner), einsum
    to_m, SO2_Convolution, einsum, bmm(wigner_inv), index_add_), fp32 torch on
    the host cores, forward + backward, on the first molecules of config 2."""
    import numpy as np
    import torch
    from oracle import message as omsg
    from oracle import rotation as orot
    from maloq_amd import synth

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = synth.config2_graph()
    L, Mm, C = 4, 2, 128
    gen = torch.Generator().manual_seed(0)
    Jd = orot.load_jd(torch.float32)
    conv = {"w0": torch.randn(5 * C, 5 * C, generator=gen) / math.sqrt(5 * C),
            "b0": torch.zeros(5 * C),
            "wm": [torch.randn(2 * (L - m + 1) * C, (L - m + 1) * C, generator=gen) / math.sqrt((L - m + 1) * C)
                   for m in (1, 2)], "c_out": C}
    for k in ("w0", "b0"):
        conv[k].requires_grad_()
    for wmm in conv["wm"]:
        wmm.requires_grad_()
    # the reference's RadialMLP as torch modules (radial.py:115-142), fp32 CPU
    torch.manual_seed(0)
    radial = torch.nn.Sequential(torch.nn.Linear(8, 64), torch.nn.LayerNorm(64), torch.nn.SiLU(),
                                 torch.nn.Linear(64, 64), torch.nn.LayerNorm(64), torch.nn.SiLU(),
                                 torch.nn.Linear(64, 1536))

    def run(nmol):
        sel = np.isin(g.mol[g.dst], np.arange(nmol))
        nodes = np.nonzero(np.isin(g.mol, np.arange(nmol)))[0]
        ei = torch.from_numpy(np.stack([g.src[sel], g.dst[sel]]))
        vec = torch.from_numpy(g.edge_distance_vec()[sel]).float()
        x = torch.randn(len(nodes), 25, C, generator=gen).requires_grad_()
        t0 = time.perf_counter()
        rad = radial(gaussian_rbf(vec.norm(dim=1), 0.0, 6.0, 8))
        eul = orot.init_edge_rot_euler_angles(vec, torch.rand(len(vec), generator=gen))
        out = omsg.message_block(x, ei, eul, Jd, L, Mm, conv, rad=rad)
        out.backward(torch.ones_like(out))
        return time.perf_counter() - t0, int(sel.sum())

    run(1)  # warm-up
    t1, e1 = run(1)
    nmol = max(1, min(32, int(budget_s / 5 / max(t1, 1e-3))))
    times = []
    for _ in range(5):
        t, e = run(nmol)
        times.append(t)
    t = sorted(times)[len(times) // 2]
    return {"value": e / t, "unit": "edges/s", "cores": cores, "kind": "port",
            "sample": f"config 2, first {nmol} molecule(s) ({e} edges), fp32 torch CPU, fwd+bwd, median of 5",
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
        lab = np.zeros((len(r), 196), np.float32)
        om2l.single_matrix2label(t.orbital_template, off, z, r, c, H, lab, True)
        o.get_net_out(torch.from_numpy(lab))
        total_t += time.perf_counter() - t0
        total_blocks += len(r)
        if total_t > budget_s:
            break
    return {"value": total_blocks / total_t, "unit": "H-blocks/s", "cores": cores, "kind": "port",
            "sample": f"config 3, {m + 1} molecule(s) ({total_blocks} blocks), numpy gather + fp32 matmul"}


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


def torch_randn_like_nodes(ew):
    import torch
    gen = torch.Generator().manual_seed(7)
    return torch.randn(ew["x"].shape, generator=gen).to(ew["x"].device)


def profile_only(args):
    """Runs one piece of the path --reps times (for rocprofv3 passes)."""
    import torch
    if args.only == "copy":
        # plain copy of a known size: calibrates FETCH_SIZE / WRITE_SIZE
        a = torch.ones(64 * 1024 * 1024, device="cuda")
        b = torch.empty_like(a)
        for _ in range(args.reps):
            b.copy_(a)
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
    elif args.only in ("fwd", "step"):
        w = message_workload(args.dtype)
        if args.only == "fwd":
            fused_forward_launch_time(w, reps=args.reps)
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
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "fp32"])
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--no-extras", action="store_true", help="headline only")
    ap.add_argument("--only", choices=["fwd", "step", "basis", "copy", "embed", "edgewise", "edgewise-step"],
                    help="profiling mode: run one piece a few times and exit (no JSON line)")
    ap.add_argument("--reps", type=int, default=5, help="launches in --only mode")
    ap.add_argument("--traffic-from", metavar="DIR",
                    help="write profiles/traffic.json from rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE runs in DIR")
    args = ap.parse_args(argv)
    if args.traffic_from:
        return traffic_from(args.traffic_from, args.dtype)
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
    if not args.no_extras:
        if args.dtype == "bf16":
            w32 = message_workload("fp32")
            t32 = time_steps(lambda: message_step(w32, True), max(3, args.steps // 4), 2)
            result["fp32_fwd_bwd_edges_per_s"] = w32["E"] / t32
            tl32 = fused_forward_launch_time(w32, reps=5)
            result["fp32_fwd_roofline_frac"] = f_edge * w32["E"] / tl32 / PEAK_FP32
            del w32
        print("[bench] basis transform (config 3) ...", file=sys.stderr, flush=True)
        bw = basis_workload()
        tf, ti, rt, tplan = basis_timing(bw)
        bpb = (bw["block_bytes"] + 4 * bw["T"] * bw["n_blocks"]) / bw["n_blocks"]
        result["basis_transform"] = {
            "metric": "H-blocks/s", "fwd": bw["n_blocks"] / tf, "inv": bw["n_blocks"] / ti,
            "blocks": bw["n_blocks"], "round_trip_rel_err": rt, "plan_ms": tplan * 1e3,
            "roofline": {"bound": "hbm", "achieved": bpb * bw["n_blocks"] / tf / 1e9, "peak": PEAK_HBM / 1e9,
                         "unit": "GB/s", "frac": bpb * bw["n_blocks"] / tf / PEAK_HBM,
                         "bytes_per_block": bpb, "traffic": load_traffic("fock_to_irreps")},
        }
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
