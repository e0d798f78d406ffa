"""Liveness-based buffer reuse (torch_helion/hip/memplan.py), on the CPU: the allocator
never hands a block to a tensor while an earlier tensor in it is still to be read, and a
deep program needs far fewer bytes than one buffer per tensor."""

from __future__ import annotations

import math

import torch


def _program(n_layers: int, tmp_path):
    from targets.mamba import MambaConfig, build_mamba_model
    from torch_helion import CompileConfig, compile_model

    cfg = MambaConfig(batch=1, seq=64, d_model=64, expand=2, headdim=16, d_state=16, chunk=32, n_layers=n_layers,
                      ngroups=1, use_conv=True, dtype=torch.bfloat16, a_log_range=(0.0, math.log(16.0)), vocab=300)
    m = build_mamba_model(cfg, seed=0)
    ids = m.example_inputs(seed=0)[0]
    res = compile_model(m, (ids,), CompileConfig(run_name="mp", results_dir=tmp_path, backend="none",
                                                 planner_mode="greedy", reference_check=False, verify_passes=False))
    return res.program


def _replay(program, pool):
    """Bind every kernel's outputs in program order as DeviceProgram does; return
    {tensor: block} and check no block is shared by tensors whose lifetimes overlap."""
    from torch_helion.hip.memplan import lifetimes

    born, last = lifetimes(program)
    holder: dict[int, tuple[str, int]] = {}
    where = {}
    for i, k in enumerate(program.kernels):
        pool.release_before(i)
        for o in k.outputs:
            t = program.tensors[o.tensor]
            nbytes = math.prod(t.shape) * 2
            blk = pool.alloc(nbytes, last[o.tensor])
            prev = holder.get(id(blk))
            assert prev is None or prev[1] < i, (o.tensor, "reuses the block of", prev[0], "still read at", prev[1])
            assert blk.numel() >= nbytes
            holder[id(blk)] = (o.tensor, last[o.tensor])
            where[o.tensor] = blk
        # every argument of kernel i is still in the block it was given
        for a in k.args:
            if a.tensor in where:
                assert holder[id(where[a.tensor])][0] == a.tensor, (k.name, a.tensor)
    return where


def test_lifetimes_cover_every_read(tmp_path):
    from torch_helion.hip.memplan import lifetimes

    prog = _program(2, tmp_path)
    born, last = lifetimes(prog)
    for i, k in enumerate(prog.kernels):
        for a in k.args:
            assert last[a.tensor] >= i
        for o in k.outputs:
            assert born[o.tensor] <= i <= last[o.tensor]
    for o in prog.outputs:
        assert last[o] == len(prog.kernels)


def test_pool_never_overlaps_live_tensors_and_saves_memory(tmp_path):
    from torch_helion.hip.memplan import BufferPool

    prog = _program(6, tmp_path)
    pool = BufferPool(lambda n: torch.empty(n, dtype=torch.uint8))
    _replay(prog, pool)
    # six layers of identically shaped activations fit in about one layer's worth of blocks
    assert pool.block_bytes < 0.4 * pool.requested_bytes, (pool.block_bytes, pool.requested_bytes)


def test_pool_best_fit_and_release_order():
    from torch_helion.hip.memplan import BufferPool

    made = []
    pool = BufferPool(lambda n: made.append(n) or torch.empty(n, dtype=torch.uint8))
    a = pool.alloc(1000, last=0)      # dies after kernel 0
    b = pool.alloc(5000, last=2)
    pool.release_before(1)            # frees a only
    c = pool.alloc(900, last=3)       # fits a's block
    assert c is a and made == [1024, 5120]
    d = pool.alloc(2000, last=3)      # nothing free that fits: new block
    assert d is not b and made == [1024, 5120, 2048]
    pool.release_before(3)            # frees b (last read by kernel 2)
    e = pool.alloc(4096, last=4)
    assert e is b


def test_conv_merge_groups_one_per_layer(tmp_path):
    """Each Mamba-2 layer's x, B and C convolutions form one group (one launch over the
    xBC channels side by side), whose members all feed that layer's SSD, with the
    SSD after the group's last member; a conv whose input or output must keep its
    own buffer (fp32 copy, program output) stays out."""
    from torch_helion.hip.runtime import conv_merge_groups

    program = _program(3, tmp_path)
    kern = {k.name: k for k in program.kernels}
    index = {k.name: i for i, k in enumerate(program.kernels)}
    convs = [k.name for k in program.kernels if k.kind == "conv1d"]
    groups = conv_merge_groups(program)
    assert len(groups) == 3 and sorted(n for g in groups for n in g) == sorted(convs)
    widths = sorted(program.tensors[kern[n].arg("x").tensor].shape[1] for n in groups[0])
    assert widths == [16, 16, 128]  # B and C (ngroups x d_state), x (d_inner)
    for g in groups:
        ys = {kern[n].outputs[0].tensor for n in g}
        ssd = [k for k in program.kernels if k.kind.startswith("ssd") and ys & {a.tensor for a in k.args}]
        assert len(ssd) == 1 and ys <= {a.tensor for a in ssd[0].args}
        assert index[ssd[0].name] > max(index[n] for n in g)
    # an excluded input (say, one with an fp32 copy) keeps its conv out of the group
    x0 = kern[groups[0][0]].arg("x").tensor
    g2 = conv_merge_groups(program, {x0})
    assert len(g2) == 3 and groups[0][0] not in [n for g in g2 for n in g]
