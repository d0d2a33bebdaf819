"""Two ranks over gloo (CPU tensors) drive the tensor-parallel forward
plumbing end to end with the dense linear method: a checkpoint stream is
sharded and merged per rank (weight_loader.py:40-69, :121-142), a gated MLP
runs as a merged column-parallel gate_up projection, silu_and_mul and a
row-parallel down projection whose partial outputs are all-reduced
(linear.py:127-143, :171-194), and an attention output projection as a
row-parallel layer.  Every rank's output must equal the single-process
forward of the unsharded weights."""

import os
import socket

import torch
import torch.distributed as dist
import torch.multiprocessing as mp

H, I, HEADS, D, T = 64, 96, 4, 16, 5


def _checkpoint(seed: int):
    g = torch.Generator().manual_seed(seed)
    w = lambda n, k: torch.randn((n, k), generator=g) * 0.1  # noqa: E731
    return [("model.layers.0.mlp.gate_proj.weight", w(I, H)), ("model.layers.0.mlp.up_proj.weight", w(I, H)),
            ("model.layers.0.mlp.down_proj.weight", w(H, I)), ("model.layers.0.self_attn.o_proj.weight", w(H, HEADS * D))]


def _reference(ckpt, x, attn):
    d = dict(ckpt)
    pre = "model.layers.0."
    gate = x @ d[pre + "mlp.gate_proj.weight"].T
    up = x @ d[pre + "mlp.up_proj.weight"].T
    mlp = (torch.nn.functional.silu(gate) * up) @ d[pre + "mlp.down_proj.weight"].T
    o = attn @ d[pre + "self_attn.o_proj.weight"].T
    return mlp, o


def _rank(rank: int, world: int, port: int, q) -> None:
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        from sglite_amd import checkpoint
        from sglite_amd.linear import MergedColumnParallelLinear, RowParallelLinear

        ckpt = _checkpoint(seed=3)
        g = torch.Generator().manual_seed(4)
        x = torch.randn((T, H), generator=g)
        attn = torch.randn((T, HEADS * D), generator=g)
        shards = dict(checkpoint.ingest(ckpt, rank=rank, world=world))
        pre = "model.layers.0."
        gate_up = MergedColumnParallelLinear(H, [I, I], False, tp_size=world)
        down = RowParallelLinear(I, H, False, tp_size=world)
        o_proj = RowParallelLinear(HEADS * D, H, False, tp_size=world)
        gate_up.load_state_dict({"weight": shards[pre + "mlp.gate_up_proj.weight"]})
        down.load_state_dict({"weight": shards[pre + "mlp.down_proj.weight"]})
        o_proj.load_state_dict({"weight": shards[pre + "self_attn.o_proj.weight"]})
        h = gate_up(x)  # this rank's gate and up columns
        li = I // world
        act = torch.nn.functional.silu(h[:, :li]) * h[:, li:]
        mlp = down(act)  # all-reduced over the ranks
        per = HEADS * D // world
        o = o_proj(attn[:, rank * per:(rank + 1) * per].contiguous())
        ref_mlp, ref_o = _reference(ckpt, x, attn)
        q.put((rank, float((mlp - ref_mlp).abs().max()), float((o - ref_o).abs().max()),
               float(ref_mlp.abs().max()), tuple(h.shape)))
    finally:
        dist.destroy_process_group()


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def test_two_rank_gated_mlp_and_row_parallel_all_reduce():
    world = 2
    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    port = _free_port()
    procs = [ctx.Process(target=_rank, args=(r, world, port, q)) for r in range(world)]
    for p in procs:
        p.start()
    res = [q.get(timeout=120) for _ in range(world)]
    for p in procs:
        p.join(timeout=60)
        assert p.exitcode == 0
    for rank, err_mlp, err_o, mx, hshape in sorted(res):
        assert hshape == (T, 2 * I // world)  # N / tp columns per rank, gate and up halves
        assert err_mlp <= 1e-5 * max(1.0, mx), (rank, err_mlp)
        assert err_o <= 1e-5, (rank, err_o)
