"""Expert slot uploads (the device side of copy_slot, crates/model/src/experts.rs:1880-1893): raw slabs
of host slots into device slot tensors, through the kernel engine (workgroups reading pinned host memory)
and the copy engines. Bytes must arrive exactly; the step run on the slots must equal the step run on
the full expert tensors; bad slot lists are refused before anything is written (the reference's
check_range, crates/ggml-sys/src/ggml/context.rs:593-609)."""
import sys

import numpy as np
import pytest
import torch

from tetraeder_amd import ggml
from tests.helpers import normal
from tests.test_gpu_mmid import make_experts, qwen3_moe_ids

pytestmark = pytest.mark.gpu

N_EMBD, N_FF = 2048, 768


def _case(name):
    print(f"[slots] {name}", file=sys.stderr, flush=True)


def _host_slabs(n_slots, seed, pinned=True):
    """gate, up (Q4_K [2048, 768, n]) and down (Q6_K [768, 2048, n]) of random bytes in host memory."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for ty, k, n in ((ggml.Type.Q4_K, N_EMBD, N_FF), (ggml.Type.Q4_K, N_EMBD, N_FF), (ggml.Type.Q6_K, N_FF, N_EMBD)):
        nbytes = ty.row_size(k) * n * n_slots
        buf = torch.empty(nbytes, dtype=torch.uint8, pin_memory=pinned)
        buf.copy_(torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g))
        out.append(ggml.QTensor(ty, (k, n, n_slots), buf))
    return out


def _device_slots(like, n_slots, device, fill=0xA5):
    return [ggml.QTensor(t.type, (t.ne[0], t.ne[1], n_slots),
                         torch.full((t.nb[2] * n_slots,), fill, dtype=torch.uint8, device=device)) for t in like]


def _slab(t, slot):
    return t.data[t.nb[2] * slot: t.nb[2] * (slot + 1)]


@pytest.mark.parametrize("engine", [ggml.COPY_KERNEL, ggml.COPY_DMA, ggml.COPY_AUTO])
def test_slabs_arrive_exactly(gpu, engine):
    """Five experts from 12 host slots to 8 device slots; the three other device slots keep their bytes."""
    _case(f"bytes engine={engine}")
    src = _host_slabs(12, seed=engine)
    dst = _device_slots(src, 8, gpu)
    frm, to = [3, 0, 11, 5, 7], [6, 1, 0, 2, 7]
    ggml.copy_expert_slots(src, dst, frm, to, engine=engine)
    torch.cuda.synchronize()
    for s, d in zip(src, dst):
        for f, t in zip(frm, to):
            assert torch.equal(_slab(d, t).cpu(), _slab(s, f)), f"slot {f} -> {t} differs"
        for t in (3, 4, 5):
            assert bool((_slab(d, t) == 0xA5).all()), f"untouched slot {t} was written"


def test_pageable_sources(gpu):
    """The copy engines take pageable host memory; the kernel engine refuses it (it reads pinned memory
    only), and the automatic choice falls back to the copy engines."""
    _case("pageable sources")
    src = _host_slabs(4, seed=9, pinned=False)
    dst = _device_slots(src, 4, gpu)
    with pytest.raises(ggml.Compute):
        ggml.copy_expert_slots(src, dst, [1], [2], engine=ggml.COPY_KERNEL)
    for engine in (ggml.COPY_DMA, ggml.COPY_AUTO):
        ggml.copy_expert_slots(src, dst, [1, 3], [2, 0], engine=engine)
        torch.cuda.synchronize()
        for s, d in zip(src, dst):
            assert torch.equal(_slab(d, 2).cpu(), _slab(s, 1)) and torch.equal(_slab(d, 0).cpu(), _slab(s, 3))


def test_bad_slot_lists_are_refused(gpu):
    """Slots past either tensor, a device slot written twice, a slab layout that differs, a device-side
    source: refused, nothing written. An empty list is a no-op."""
    _case("bad slot lists")
    src = _host_slabs(4, seed=3)
    dst = _device_slots(src, 4, gpu)
    for frm, to in (([4], [0]), ([0], [4]), ([0, 1], [2, 2])):
        with pytest.raises(ggml.Compute):
            ggml.copy_expert_slots(src, dst, frm, to)
    other = [ggml.QTensor(ggml.Type.Q6_K, (N_EMBD, N_FF, 4), torch.zeros(ggml.Type.Q6_K.row_size(N_EMBD) * N_FF * 4,
                                                                          dtype=torch.uint8, device=gpu))]
    with pytest.raises(ggml.Compute):
        ggml.copy_expert_slots(src[:1], other, [0], [0])
    with pytest.raises(ggml.Invalid):
        ggml.copy_expert_slots(dst, dst, [0], [1])
    ggml.copy_expert_slots(src, dst, [], [])
    torch.cuda.synchronize()
    for d in dst:
        assert bool((d.data == 0xA5).all()), "a refused call wrote a slot"


@pytest.mark.parametrize("engine", [ggml.COPY_KERNEL, ggml.COPY_DMA])
@pytest.mark.parametrize("tokens", [1, 4])
def test_slots_feed_the_moe_step(gpu, engine, tokens):
    """Qwen3-30B-A3B experts kept in pinned host memory; the routed ones are uploaded to 32 device slots
    (in expert order, so the step deals its workgroups as on the full tensors) and the step on the slots
    with the ids mapped to slots equals, bit for bit, the step on the full 128-expert tensors."""
    _case(f"moe on slots engine={engine} T={tokens}")
    E = 128
    full = [make_experts(ggml.Type.Q4_K, N_EMBD, N_FF, E, seed=71, device=gpu),
            make_experts(ggml.Type.Q4_K, N_EMBD, N_FF, E, seed=72, device=gpu),
            make_experts(ggml.Type.Q6_K, N_FF, N_EMBD, E, seed=73, device=gpu)]
    host = []
    for t in full:
        buf = torch.empty(t.data.numel(), dtype=torch.uint8, pin_memory=True)
        buf.copy_(t.data.cpu())
        host.append(ggml.QTensor(t.type, t.ne, buf))
    ids = qwen3_moe_ids(tokens, seed=900 + tokens)
    routed = sorted({int(e) for e in ids.ravel() if e >= 0})
    slot_of = {e: i for i, e in enumerate(routed)}
    slots = _device_slots(full, 32, gpu, fill=0)
    ggml.copy_expert_slots(host, slots, routed, list(range(len(routed))), engine=engine)
    slot_ids = np.vectorize(lambda e: slot_of.get(int(e), -1))(ids).astype(np.int32)
    x = torch.from_numpy(normal((tokens, 1, N_EMBD), 950 + tokens)).to(gpu)
    w = torch.from_numpy(np.random.default_rng(tokens).random((tokens, 8, 1)).astype(np.float32)).to(gpu)
    want = ggml.moe_ffn_sum(*full, x, torch.from_numpy(ids).to(gpu), w)
    got = ggml.moe_ffn_sum(*slots, x, torch.from_numpy(slot_ids).to(gpu), w)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert ggml.moe_sync_errors(clear=True) == 0


def test_kernel_upload_in_a_graph(gpu):
    """The kernel engine captured in a HIP graph reads the host bytes at each replay: new host contents
    between replays arrive in the slots."""
    _case("kernel upload in a graph")
    src = _host_slabs(6, seed=21)
    dst = _device_slots(src, 4, gpu)
    frm, to = [5, 2], [0, 3]
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        ggml.copy_expert_slots(src, dst, frm, to, engine=ggml.COPY_KERNEL)
    gen = torch.Generator().manual_seed(5)
    for r in range(3):
        for s in src:
            s.data.copy_(torch.randint(0, 256, (s.data.numel(),), dtype=torch.uint8, generator=gen))
        for d in dst:
            d.data.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for s, d in zip(src, dst):
            for f, t in zip(frm, to):
                assert torch.equal(_slab(d, t).cpu(), _slab(s, f)), f"replay {r}: slot {f} -> {t} differs"
