"""GPU test of the ops composed into one decoder layer's decode step.

fused_add_rms_norm -> qkv gemm_tn -> rotary_embedding on the q and k columns
of the qkv output -> reshape_and_cache of the new token's k and v columns ->
paged_attention_decode (q is a strided view of the qkv output, as a serving
engine passes it) -> o gemm_tn -> fused_add_rms_norm -> gate_up gemm_tn ->
silu_and_mul -> down gemm_tn, at the head-dim-256 / group-8 attention shape,
with a reduced MLP width (1024) and, as BASELINE.json's C5 names it, at full
size (256 sequences of log-uniform lengths up to 32768, Llama-3-8B's MLP width
14336; the GEMMs there are checked against an fp32 GEMM on the GPU). ``seq_lens`` counts the new token, which sits at
position len - 1; an empty sequence is a padding row (position and slot -1).
Each stage is checked against the oracle applied to the previous stage's
actual output (the bar of each op's own parity test), then the whole step is
captured in a HIP graph and every replay -- with the sequence lengths,
positions and slots rewritten on the device between replays -- must match an
eager run bit for bit. Each test also runs with rotary_embedding_and_cache in
place of the two ops, which must give the same bits.
"""

import pytest
import torch

import decodekernels_amd as dk
from decodekernels_amd.testing import make_paged_kv
from oracle.rope_cache import reshape_and_cache_reference, rope_cos_sin_cache, rotary_embedding_reference
from parity import (
    assert_max_abs,
    assert_ulp,
    attention_f32,
    fused_add_rms_norm_reference,
    gemm_f32,
    gemm_f32_gpu,
    silu_and_mul_reference,
)

pytestmark = pytest.mark.gpu

HQ, HKV, D, BS = 16, 2, 256, 32
HIDDEN, INTER = HQ * D, 1024
EPS = 1e-5


class Layer:
    def __init__(self, seq_lens, dtype, seed=0, fused_rope_cache=False, inter=INTER, fused_gemm=False):
        self.fused_rope_cache = fused_rope_cache
        self.fused_gemm = fused_gemm  # qkv gemm + rope / cache and o gemm + norm as the fused ops
        g = torch.Generator(device="cuda").manual_seed(seed)
        kw = dict(device="cuda", dtype=dtype)
        self.dtype = dtype
        self.n = len(seq_lens)
        self.w_qkv = torch.randn((HQ + 2 * HKV) * D, HIDDEN, generator=g, **kw) * 0.02
        self.w_o = torch.randn(HIDDEN, HIDDEN, generator=g, **kw) * 0.02
        self.w_gu = torch.randn(2 * inter, HIDDEN, generator=g, **kw) * 0.02
        self.w_down = torch.randn(HIDDEN, inter, generator=g, **kw) * 0.02
        self.ln1 = (1 + 0.1 * torch.randn(HIDDEN, generator=g, device="cuda")).to(dtype)
        self.ln2 = (1 + 0.1 * torch.randn(HIDDEN, generator=g, device="cuda")).to(dtype)
        self.kv = make_paged_kv(seq_lens, HKV, D, BS, dtype, "cuda", layout="nhd", seed=seed + 1)
        self.max_len = max(max(seq_lens), 1)
        self.x0 = torch.randn(self.n, HIDDEN, generator=g, **kw)
        self.r0 = torch.randn(self.n, HIDDEN, generator=g, **kw)
        self.x, self.resid = torch.empty_like(self.x0), torch.empty_like(self.r0)
        self.qkv = torch.empty(self.n, self.w_qkv.shape[0], **kw)
        self.attn = torch.empty(self.n, HQ, D, **kw)
        self.o = torch.empty(self.n, HIDDEN, **kw)
        self.gu = torch.empty(self.n, 2 * inter, **kw)
        self.act = torch.empty(self.n, inter, **kw)
        self.down = torch.empty(self.n, HIDDEN, **kw)
        self.ws = dk.alloc_workspace(self.n, HQ, D, self.max_len, "cuda")
        self.q = self.qkv[:, : HQ * D].view(self.n, HQ, D)
        self.k_new = self.qkv[:, HQ * D : (HQ + HKV) * D]
        self.v_new = self.qkv[:, (HQ + HKV) * D :]
        self.rope = rope_cos_sin_cache(max(4096, self.max_len), D, base=1e6).cuda()
        self.positions = torch.empty(self.n, dtype=torch.long, device="cuda")
        self.slots = torch.empty(self.n, dtype=torch.long, device="cuda")
        self.set_lens(seq_lens)
        self.saved = {}

    def set_lens(self, lens):
        """Lengths, positions and cache slots of a step whose new token is the
        last of each sequence (written in place: a captured graph follows)."""
        bt = self.kv.block_tables.cpu()
        pos = [n - 1 for n in lens]
        slots = [int(bt[s, p // BS]) * BS + p % BS if p >= 0 else -1 for s, p in enumerate(pos)]
        self.kv.seq_lens.copy_(torch.tensor(lens, dtype=torch.int32))
        self.positions.copy_(torch.tensor(pos))
        self.slots.copy_(torch.tensor(slots))

    def step(self, keep=False):
        ops = torch.ops.decode_kernels
        self.x.copy_(self.x0)
        self.resid.copy_(self.r0)
        ops.fused_add_rms_norm(self.x, self.resid, self.ln1, EPS)
        if keep:
            self.saved["norm1"] = (self.x.clone(), self.resid.clone())
        if self.fused_gemm:
            ops.gemm_tn_rotary_embedding_and_cache(self.qkv, self.x, self.w_qkv, None, self.positions,
                                                   self.qkv[:, : HQ * D], self.k_new, self.v_new, D, self.rope, True,
                                                   self.kv.k_cache, self.kv.v_cache, self.slots)
        else:
            ops.gemm_tn(self.qkv, self.x, self.w_qkv, None)
        if keep:
            self.saved["qkv"] = self.qkv.clone()
        if self.fused_gemm:
            pass
        elif self.fused_rope_cache:
            if keep:
                self.saved["k_cache"] = self.kv.k_cache.clone()
                self.saved["v_cache"] = self.kv.v_cache.clone()
            ops.rotary_embedding_and_cache(self.positions, self.qkv[:, : HQ * D], self.k_new, self.v_new, D,
                                           self.rope, True, self.kv.k_cache, self.kv.v_cache, self.slots)
        else:
            ops.rotary_embedding(self.positions, self.qkv[:, : HQ * D], self.k_new, D, self.rope, True)
            if keep:
                self.saved["k_cache"] = self.kv.k_cache.clone()
                self.saved["v_cache"] = self.kv.v_cache.clone()
            ops.reshape_and_cache(self.k_new, self.v_new, self.kv.k_cache, self.kv.v_cache, self.slots)
        dk.paged_attention_decode(self.q, self.kv.k_cache, self.kv.v_cache, self.kv.block_tables, self.kv.seq_lens,
                                  max_seq_len=self.max_len, out=self.attn, workspace=self.ws)
        if self.fused_gemm:
            ops.gemm_tn_add_rms_norm(self.o, self.attn.view(self.n, HIDDEN), self.w_o, None, self.resid, self.ln2, EPS)
        else:
            ops.gemm_tn(self.o, self.attn.view(self.n, HIDDEN), self.w_o, None)
            if keep:
                self.saved["o"] = self.o.clone()
                self.saved["resid1"] = self.resid.clone()
            ops.fused_add_rms_norm(self.o, self.resid, self.ln2, EPS)
        ops.gemm_tn(self.gu, self.o, self.w_gu, None)
        ops.silu_and_mul(self.act, self.gu)
        ops.gemm_tn(self.down, self.act, self.w_down, None)

    def outputs(self):
        return [t.clone() for t in (self.qkv, self.kv.k_cache, self.kv.v_cache, self.attn, self.o, self.resid, self.gu,
                                    self.act, self.down)]


SEQ_LENS = [0, 1, 600, 1500, 33, 2049, 512, 513]


def _gemm_f32_gpu(a, b):
    """fp32 GEMM on the GPU (the reference for GEMMs too large for the CPU oracle in a test)."""
    return gemm_f32_gpu(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("fused", [False, True])
def test_layer_step_stages_match_oracle(dtype, fused):
    L = Layer(SEQ_LENS, dtype, fused_rope_cache=fused)
    L.step(keep=True)
    torch.cuda.synchronize()
    _check_stages(L, dtype, gemm_f32)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_layer_step_full_width_c5(dtype):
    """BASELINE.json's C5 step at full size: 256 sequences (lengths log-uniform
    in [1, 32768], 8 empty), 16 query / 2 KV heads of 256, block 32, hidden 4096,
    MLP 2 x 14336; every stage against its oracle."""
    import math

    g = torch.Generator().manual_seed(5)
    lens = torch.exp(torch.rand(256, generator=g) * math.log(32768)).long().clamp(1, 32768)
    lens[torch.randperm(256, generator=g)[:8]] = 0
    L = Layer(lens.tolist(), dtype, seed=11, fused_rope_cache=True, inter=14336)
    L.step(keep=True)
    torch.cuda.synchronize()
    _check_stages(L, dtype, _gemm_f32_gpu)


def _check_stages(L, dtype, gemm_ref):
    x1, r1 = L.saved["norm1"]
    want_x, want_r = fused_add_rms_norm_reference(L.x0.cpu(), L.r0.cpu(), L.ln1.cpu(), EPS)
    assert torch.equal(r1.cpu(), want_r), "residual of the first fused_add_rms_norm is not bit-exact"
    assert_ulp(x1, want_x, 1, "fused_add_rms_norm")
    qkv = L.saved["qkv"]
    assert_max_abs(qkv, gemm_ref(x1, L.w_qkv), dtype, "qkv gemm")
    hq_d, kv_d = HQ * D, (HQ + HKV) * D
    want_q, want_k = rotary_embedding_reference(L.positions.cpu(), qkv[:, :hq_d].cpu(), qkv[:, hq_d:kv_d].cpu(), D,
                                                L.rope.cpu(), True)
    assert_ulp(L.qkv[:, :hq_d], want_q, 0, "rotary_embedding(q)")
    assert_ulp(L.qkv[:, hq_d:kv_d], want_k, 0, "rotary_embedding(k)")
    assert torch.equal(L.qkv[:, kv_d:], qkv[:, kv_d:]), "v columns must pass through RoPE untouched"
    want_kc, want_vc = reshape_and_cache_reference(L.k_new.cpu(), L.v_new.cpu(), L.saved["k_cache"].cpu(),
                                                   L.saved["v_cache"].cpu(), L.slots.cpu())
    assert torch.equal(L.kv.k_cache.cpu(), want_kc) and torch.equal(L.kv.v_cache.cpu(), want_vc)
    ref_attn = attention_f32(L.q, L.kv.k_cache, L.kv.v_cache, L.kv.block_tables, L.kv.seq_lens)
    assert_max_abs(L.attn, ref_attn, dtype, "attention on the qkv view")
    assert (L.attn[L.kv.seq_lens == 0] == 0).all(), "zero-length sequences must give zeros"
    assert_max_abs(L.saved["o"], gemm_ref(L.attn.view(L.n, HIDDEN), L.w_o), dtype, "o gemm")
    want_o, want_r2 = fused_add_rms_norm_reference(L.saved["o"].cpu(), L.saved["resid1"].cpu(), L.ln2.cpu(), EPS)
    assert torch.equal(L.resid.cpu(), want_r2)
    assert_ulp(L.o, want_o, 1, "second fused_add_rms_norm")
    assert_max_abs(L.gu, gemm_ref(L.o, L.w_gu), dtype, "gate_up gemm")
    assert_ulp(L.act, silu_and_mul_reference(L.gu.cpu()), 1, "silu_and_mul")
    assert_max_abs(L.down, gemm_ref(L.act, L.w_down), dtype, "down gemm")


@pytest.mark.parametrize("fused", [False, True])
def test_layer_step_graph_replays_match_eager(fused):
    dtype = torch.bfloat16
    L = Layer(SEQ_LENS, dtype, seed=3, fused_rope_cache=fused)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        L.step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        L.step()
    lens_sets = [SEQ_LENS, [5, 0, 2049, 17, 1024, 1, 700, 2000], SEQ_LENS]
    for i, lens in enumerate(lens_sets):
        L.set_lens(lens)
        graph.replay()
        torch.cuda.synchronize()
        got = L.outputs()
        L.step()
        torch.cuda.synchronize()
        want = L.outputs()
        names = ("qkv", "k_cache", "v_cache", "attn", "o", "resid", "gate_up", "act", "down")
        for name, a, b in zip(names, got, want):
            assert torch.equal(a, b), f"replay {i}: {name} differs from the eager step"


def test_layer_step_fused_gemms_equal_unfused():
    """64 sequences (decode batch 64, the shapes whose GEMM plans split K): the
    step with the qkv GEMM fused into rotary_embedding_and_cache and the o GEMM
    fused into the post-attention norm gives the same bits as the unfused step,
    and so does a graph replay of it."""
    from decodekernels_amd import capi

    g = torch.Generator().manual_seed(8)
    lens = [int(x) for x in torch.randint(1, 3000, (64,), generator=g)]
    lens[5] = 0
    assert capi.gemm_plan(64, (HQ + 2 * HKV) * D, HIDDEN)[2] > 1 and capi.gemm_plan(64, HIDDEN, HIDDEN)[2] > 1
    a = Layer(lens, torch.bfloat16, seed=9)
    b = Layer(lens, torch.bfloat16, seed=9, fused_gemm=True)
    a.step()
    b.step()
    torch.cuda.synchronize()
    names = ("qkv", "k_cache", "v_cache", "attn", "o", "resid", "gate_up", "act", "down")
    want = a.outputs()
    for name, x, y in zip(names, want, b.outputs()):
        assert torch.equal(x, y), f"{name} differs between the fused-GEMM and the unfused step"
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        b.step()
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(graph):
        b.step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name, x, y in zip(names, want, b.outputs()):
            assert torch.equal(x, y), f"{name} differs in a replay of the fused-GEMM step"


def test_layer_step_fused_rope_cache_equals_two_ops():
    """The step with rotary_embedding_and_cache gives the same bits as with
    rotary_embedding + reshape_and_cache."""
    a = Layer(SEQ_LENS, torch.bfloat16, seed=5)
    b = Layer(SEQ_LENS, torch.bfloat16, seed=5, fused_rope_cache=True)
    a.step()
    b.step()
    torch.cuda.synchronize()
    names = ("qkv", "k_cache", "v_cache", "attn", "o", "resid", "gate_up", "act", "down")
    for name, x, y in zip(names, a.outputs(), b.outputs()):
        assert torch.equal(x, y), f"{name} differs between the fused and the two-op step"
