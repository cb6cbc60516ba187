"""GPU parity of the drop-in ``swamla_amd.MLA`` against the reference:
the golden fixtures written by the real reference, and the oracle's op-for-op
restatement (oracle/mla_ref.py) on identical seeded inputs and weights.

Bars: attention outputs within 2e-2 relative / 1e-2 absolute (bf16) and
1e-4 / 1e-5 (fp32); cache rows bit-exact given the wkv_a rows: latent rows
equal torch's CPU LayerNorm (the reference's kv_norm) bit for bit, k_pe rows
the per-op-rounded RoPE."""
import glob
import hashlib
import os

import pytest
import torch

from oracle import latent_ops as lo
from oracle.mla_ref import MLAConfig, RefMLA, enable_cache, init_weights
from swamla_amd import MLA, kernels

pytestmark = pytest.mark.gpu

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "mla_*.pt")))
TOL = {torch.bfloat16: (2e-2, 1e-2), torch.float32: (1e-4, 1e-5)}


def say(*a):
    print(*a, flush=True)


def close(out, ref, dtype):
    rtol, atol = TOL[dtype]
    out, ref = out.double().cpu(), ref.double().cpu()
    err = (out - ref).abs()
    bad = err > atol + rtol * ref.abs()
    assert not bool(bad.any()), f"{int(bad.sum())}/{bad.numel()} outside tol, max err {float(err.max()):.3e}"


def expected_cache(m, xs, dtype, fp8=False):
    """Oracle cache contents for the append kernel's actual inputs: the wkv_a
    rows the GPU computed in forward (recomputed with the same GEMM), put
    through torch's CPU LayerNorm order, per-op RoPE at the call-local
    positions and, for e4m3, torch's cast.  Calls are contiguous from 0."""
    cos, sin = (t.cpu() for t in m.rope.half_tables())
    w = m.kv_norm.weight.detach().cpu()
    b = m.kv_norm.bias.detach().cpu()
    rank, rpad = m.kv_lora_rank, m.rank_pad
    cs, ps, ss = [], [], []
    with torch.no_grad():
        for x in xs:
            B, T, _ = x.shape
            kv = m.input_projections(x)[1].cpu()  # the rows forward fed the append kernel
            y = lo.layernorm_aten(kv[:, :rank], w, b, m.kv_norm.eps)[0]
            # the oracle statement is torch's own CPU LayerNorm, bit for bit
            ref_ln = torch.nn.functional.layer_norm(kv[:, :rank], (rank,), w, b, m.kv_norm.eps)
            assert torch.equal(y.view(torch.uint8), ref_ln.view(torch.uint8))
            y = torch.cat([y, torch.zeros(y.shape[0], rpad - rank, dtype=y.dtype)], 1)  # zero padding
            rp = torch.arange(T).repeat(B)
            kpe = lo.rope_interleaved(kv[:, rpad:rpad + 64], cos[rp], sin[rp])
            if fp8:
                y, sc = lo.fp8_quantize(y)
                ss.append(sc.view(B, T))
            cs.append(y.view(B, T, -1))
            ps.append(kpe.view(B, T, -1))
    return torch.cat(cs, 1), torch.cat(ps, 1), (torch.cat(ss, 1) if fp8 else None)


def assert_cache_bits(m, xs, dtype, fp8=False):
    c, p, s = expected_cache(m, xs, dtype, fp8)
    B, L = c.shape[:2]
    got_c, got_p = m.kv_cache[:B, :L].cpu(), m.pe_cache[:B, :L].cpu()
    assert torch.equal(got_c.view(torch.uint8), c.view(torch.uint8)), "latent cache bits differ from the oracle"
    assert torch.equal(got_p.view(torch.uint8), p.view(torch.uint8)), "k_pe cache bits differ from the oracle"
    if fp8:
        assert torch.equal(m.kv_scale[:B, :L].cpu(), s), "e4m3 scales differ from the oracle"


def checksums(module):
    return {n: hashlib.sha256(p.detach().float().cpu().contiguous().numpy().tobytes()).hexdigest()
            for n, p in module.named_parameters()}


def make_pair(cfg, seed, dtype, gpu, ln_random=False, fp8=False):
    ref = RefMLA(cfg, fp8_cache=fp8)
    init_weights(ref, seed, ln_random=ln_random)
    ref.eval()
    enable_cache(ref)
    ref.to(dtype)
    ours = MLA(cfg, cache_dtype="fp8_e4m3" if fp8 else None)
    ours.load_state_dict(ref.state_dict())
    ours.eval().to(dtype).to(gpu)
    ours.set_inference_mode(True)
    return ref, ours


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p) for p in GOLDEN])
def test_module_matches_reference_fixtures(gpu, path):
    blob = torch.load(path, weights_only=True)
    meta = blob["meta"]
    say(f"golden {meta['name']}")
    dtype = torch.bfloat16 if "bfloat16" in meta["dtype"] else torch.float32
    cfg = MLAConfig(n_embd=meta["dim"], max_batch_size=meta["batch"], max_seq_len=meta["max_seq_len"])
    m = MLA(cfg)
    init_weights(m, meta["seed"], ln_random=meta["ln_random"])
    assert checksums(m) == blob["checksums"]
    m.eval().to(dtype).to(gpu)
    m.set_inference_mode(True)
    pos = 0
    xs = [x.to(gpu) for x in blob["inputs"]]
    masks = blob.get("masks") or [None] * len(xs)
    with torch.no_grad():
        for x, ref_out, mask in zip(xs, blob["outputs"], masks):
            out = m(x, pos, None, None if mask is None else mask.to(gpu))
            close(out, ref_out, dtype)
            pos += x.shape[1]
    torch.cuda.synchronize()
    # bit-exact against the oracle on the kernel's own inputs ...
    assert_cache_bits(m, xs, dtype)
    # ... and close to the reference's CPU-computed caches (whose wkv_a GEMM
    # rounds differently from the GPU's)
    B = meta["batch"]
    close(m.pe_cache[:B, :pos], blob["pe_cache"], dtype)
    close(m.kv_cache[:B, :pos], blob["kv_cache"], dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_config1_prefill_512_then_decode(gpu, dtype):
    """batch 1, a 512-token prefill, then its 64 decode
    steps, each output against the CPU oracle and the cache bits after the
    last step."""
    say(f"config1 dtype={dtype}")
    cfg = MLAConfig(n_embd=1024, max_batch_size=1, max_seq_len=640)
    ref, ours = make_pair(cfg, 21, dtype, gpu)
    g = torch.Generator().manual_seed(22)
    x = torch.randn(1, 512, 1024, generator=g).to(dtype)
    xs = [x.to(gpu)]
    with torch.no_grad():
        close(ours(xs[0], 0), ref(x, 0), dtype)
        for step in range(64):
            xd = torch.randn(1, 1, 1024, generator=g).to(dtype)
            xs.append(xd.to(gpu))
            close(ours(xs[-1], 512 + step), ref(xd, 512 + step), dtype)
    torch.cuda.synchronize()
    assert_cache_bits(ours, xs, dtype)
    close(ours.pe_cache[:1, :576], ref.pe_cache[:1, :576], dtype)
    close(ours.kv_cache[:1, :576], ref.kv_cache[:1, :576], dtype)


@pytest.mark.parametrize("split_plan", ["auto", "static"])
def test_per_sequence_start_pos(gpu, split_plan):
    """Ragged batch through a start_pos tensor equals each sequence run alone
    through the reference (whose interface takes one int per call), with the
    device-balanced split plan (auto, for a tensor) and the per-row one."""
    say(f"ragged start_pos, split_plan={split_plan}")
    dtype = torch.bfloat16
    cfg = MLAConfig(n_embd=256, max_batch_size=3, max_seq_len=128)
    lens = [40, 7, 90]
    g = torch.Generator().manual_seed(23)
    prompts = [torch.randn(1, L, 256, generator=g).to(dtype) for L in lens]
    step = torch.randn(3, 1, 256, generator=g).to(dtype)
    refs = []
    for i in range(3):
        r, _ = make_pair(MLAConfig(n_embd=256, max_batch_size=1, max_seq_len=128), 24, dtype, gpu)
        with torch.no_grad():
            r(prompts[i], 0)
            refs.append(r(step[i:i + 1], lens[i]))
    _, ours = make_pair(cfg, 24, dtype, gpu)
    ours.split_plan = split_plan
    with torch.no_grad():
        # fill each batch slot with its own prompt through the append path
        # (padding rows beyond a slot's length are overwritten by the step)
        maxL = max(lens)
        xpad = torch.zeros(3, maxL, 256, dtype=dtype)
        for i in range(3):
            xpad[i, : lens[i]] = prompts[i][0]
        ours.prefill_cache(xpad.to(gpu), 0)
        out = ours(step.to(gpu), torch.tensor(lens, dtype=torch.int32, device=gpu))
    close(out, torch.cat(refs), dtype)


@pytest.mark.parametrize("fused", [True, False])
def test_advance_positions(gpu, fused):
    """MLA.advance_positions: the call adds T to a start_pos tensor after its
    kernels have read it: inside wo's launch on the fused one-token path (an
    int32 device tensor), else by an in-place add.  Outputs and cache bits
    equal those of a module that does not advance (the caller adding 1), for
    several steps in a row; an int start_pos raises."""
    say(f"advance_positions fused={fused}")
    dtype = torch.bfloat16
    cfg = MLAConfig(n_embd=1024, max_batch_size=4, max_seq_len=256)
    _, a = make_pair(cfg, 31, dtype, gpu)
    _, b = make_pair(cfg, 31, dtype, gpu)
    a.advance_positions = True
    g = torch.Generator().manual_seed(32)
    prompt = torch.randn(4, 40, 1024, generator=g).to(dtype).to(gpu)
    with torch.no_grad():
        a.prefill_cache(prompt, 0)
        b.prefill_cache(prompt, 0)
        lens = [40, 33, 17, 40]
        pa = torch.tensor(lens, dtype=torch.int32, device=gpu)
        if not fused:
            pa = pa.to(torch.int64)  # not the kernels' own storage: forward adds in place
        pb = torch.tensor(lens, dtype=torch.int32, device=gpu)
        for i in range(5):
            x = torch.randn(4, 1, 1024, generator=g).to(dtype).to(gpu)
            ya = a(x, pa)
            assert a._advance_folded == fused
            yb = b(x, pb)
            pb.add_(1)
            torch.cuda.synchronize()
            assert torch.equal(ya, yb)
            assert torch.equal(pa.cpu().to(torch.int32), pb.cpu())
        assert torch.equal(pa.cpu().to(torch.int32), torch.tensor(lens, dtype=torch.int32) + 5)
        assert torch.equal(a.kv_cache.view(torch.uint8), b.kv_cache.view(torch.uint8))
        assert torch.equal(a.pe_cache.view(torch.uint8), b.pe_cache.view(torch.uint8))
        # a prompt-sized chunk advances by its length
        xs = torch.randn(4, 3, 1024, generator=g).to(dtype).to(gpu)
        a(xs, pa)
        assert not a._advance_folded
        assert torch.equal(pa.cpu().to(torch.int32), torch.tensor(lens, dtype=torch.int32) + 8)
        with pytest.raises(ValueError):
            a(x, 50)


def test_fp8_cache_against_emulation(gpu):
    """e4m3 latent cache vs the reference with the quantisation emulated in
    PyTorch (oracle RefMLA(fp8_cache=True))."""
    say("fp8 module")
    dtype = torch.bfloat16
    cfg = MLAConfig(n_embd=1024, max_batch_size=2, max_seq_len=300)
    ref, ours = make_pair(cfg, 25, dtype, gpu, ln_random=True, fp8=True)
    g = torch.Generator().manual_seed(26)
    x = torch.randn(2, 200, 1024, generator=g).to(dtype)
    xs = [x.to(gpu)]
    with torch.no_grad():
        close(ours(xs[0], 0), ref(x, 0), dtype)
        for s in range(8):
            xd = torch.randn(2, 1, 1024, generator=g).to(dtype)
            xs.append(xd.to(gpu))
            close(ours(xs[-1], 200 + s), ref(xd, 200 + s), dtype)
    torch.cuda.synchronize()
    assert_cache_bits(ours, xs, dtype, fp8=True)


def test_module_decode_batch_128(gpu):
    """128 query rows per decode step (config 5's batch): mla_linear_packed
    would need a second round of workgroups for the stacked input product, so
    the module runs that product on the library GEMM, and wo still on
    mla_linear_packed.  Against the reference restatement; cache rows
    bit-exact."""
    from swamla_amd import kernels

    say("module, batch 128 decode")
    dtype = torch.bfloat16
    B = 128
    cfg = MLAConfig(n_embd=1024, max_batch_size=B, max_seq_len=96)
    ref, ours = make_pair(cfg, 31, dtype, gpu, ln_random=True)
    ours.decode_weights()
    wp = ours._decode_w[3]  # the packed stacked weight
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    assert kernels.packed_blocks(B, wp.N, wp.K) > cus  # the routing this test covers
    g = torch.Generator().manual_seed(32)
    x = torch.randn(B, 40, 1024, generator=g).to(dtype)
    xs = [x.to(gpu)]
    with torch.no_grad():
        close(ours(xs[0], 0), ref(x, 0), dtype)
        for s in range(3):
            xd = torch.randn(B, 1, 1024, generator=g).to(dtype)
            xs.append(xd.to(gpu))
            close(ours(xs[-1], 40 + s), ref(xd, 40 + s), dtype)
    torch.cuda.synchronize()
    assert_cache_bits(ours, xs, dtype)


def test_no_cache_forward_matches_reference(gpu):
    """Outside inference mode the reference attends over the call's own
    tokens with a causal mask (mla.py:419-423, :483)."""
    say("no-cache forward")
    dtype = torch.bfloat16
    cfg = MLAConfig(n_embd=512, max_batch_size=2, max_seq_len=64)
    ref = RefMLA(cfg)
    init_weights(ref, 27)
    ref.eval().to(dtype)
    ours = MLA(cfg)
    ours.load_state_dict(ref.state_dict())
    ours.eval().to(dtype).to(gpu)
    x = torch.randn(2, 33, 512).to(dtype)
    with torch.no_grad():
        close(ours(x.to(gpu), 0), ref(x, 0), dtype)


def test_no_cache_forward_grows_rope_table_fp32(gpu):
    """An fp32 no-cache call longer than max_seq_len grows the RoPE table to
    the call's length on the module's device (positional_encoding.py:44-46,
    :64-86) and matches the restatement, which grows its table on the CPU."""
    say("no-cache forward, RoPE growth")
    cfg = MLAConfig(n_embd=256, max_batch_size=2, max_seq_len=32)
    ref = RefMLA(cfg)
    init_weights(ref, 29)
    ref.eval()
    ours = MLA(cfg)
    ours.load_state_dict(ref.state_dict())
    ours.eval().to(gpu)
    g = torch.Generator().manual_seed(30)
    x = torch.randn(2, 75, 256, generator=g)
    with torch.no_grad():
        close(ours(x.to(gpu), 0), ref(x, 0), torch.float32)
    assert ours.rope.max_seq_len == ref.rope.max_seq_len == 75
    assert ours.rope.cos_cached.device.type == "cuda"
    x2 = torch.randn(2, 40, 256, generator=g)  # within the grown table
    with torch.no_grad():
        close(ours(x2.to(gpu), 0), ref(x2, 0), torch.float32)


@pytest.mark.parametrize("rank,q_lora,dim", [
    (128, 0, 256), (173, 0, 256), (320, 0, 256), (449, 0, 256), (512, 0, 256),
    (256, 96, 256), (200, 160, 1024), (300, 0, 1024), (640, 0, 256), (1024, 0, 512), (777, 160, 256),
])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_module_any_rank_and_q_lora(gpu, dtype, rank, q_lora, dim, monkeypatch):
    """kv_lora_rank other than 256 (the real model scales it per layer:
    swa_mla_model.py:216-247, up to 1024 from SWAMLAConfig's default base of
    512, :65, :219) and the low-rank query path (mla.py:98-103):
    a prefill chunk, then decode steps at batch 2, against the reference
    restatement with the same weights; cache rows bit-exact.  bf16 decode
    steps take the fused step (a q low-rank module through its two products
    with q_norm between them)."""
    say(f"rank={rank} q_lora={q_lora} dim={dim} dtype={dtype}")
    cfg = MLAConfig(n_embd=dim, max_batch_size=2, max_seq_len=192, kv_lora_rank=rank, q_lora_rank=q_lora)
    ref, ours = make_pair(cfg, 31 + rank, dtype, gpu, ln_random=True)
    fused = []
    real_mp = kernels.merge_project
    monkeypatch.setattr(kernels, "merge_project", lambda *a, **k: (fused.append(1), real_mp(*a, **k))[1])
    assert ours.kv_cache.shape[-1] == 64 * -(-rank // 64)
    g = torch.Generator().manual_seed(32 + rank)
    x = torch.randn(2, 40, dim, generator=g).to(dtype)
    xs = [x.to(gpu)]
    with torch.no_grad():
        close(ours(xs[0], 0), ref(x, 0), dtype)
        for step in range(6):
            xd = torch.randn(2, 1, dim, generator=g).to(dtype)
            xs.append(xd.to(gpu))
            close(ours(xs[-1], 40 + step), ref(xd, 40 + step), dtype)
    torch.cuda.synchronize()
    assert_cache_bits(ours, xs, dtype)
    assert bool((ours.kv_cache[:2, :46, rank:].float() == 0).all())
    # the 80-row prompt and six steps take the fused step (ranks up to 512)
    assert len(fused) == (7 if dtype == torch.bfloat16 and rank <= 512 else 0), fused


@pytest.mark.parametrize("n_head,dim,nope,rank", [(12, 1024, 128, 256), (32, 1024, 128, 256), (8, 512, 128, 173),
                                                  (32, 1024, 64, 256)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_module_other_head_counts(gpu, dtype, n_head, dim, nope, rank, monkeypatch):
    """The reference presets' head counts (moe-1b: 12, xl: 32,
    swa_mla_model.py:618-640; 32 heads of 64 nope channels is the
    cudnn-compatible layout, :697-698): a 160-token prompt (the prompt-sized
    products), then decode steps at batch 2, against the reference
    restatement with the same weights; cache rows bit-exact.  bf16 modules
    with 32 heads run every attention call as one 32-head launch (the cache
    streamed once); other counts as 16-head launches over zero-padded query
    heads.  bf16 decode steps take the fused step, with fewer than 16 heads
    padded to 16 (zero query rows, read-out and wo columns)."""
    say(f"n_head={n_head} dim={dim} nope={nope} rank={rank} dtype={dtype}")
    cfg = MLAConfig(n_embd=dim, n_head=n_head, max_batch_size=2, max_seq_len=192, kv_lora_rank=rank,
                    qk_nope_head_dim=nope)
    ref, ours = make_pair(cfg, 41 + n_head, dtype, gpu, ln_random=True)
    calls = []
    real = kernels.decode_attention

    def spy(q_abs, *a, **k):
        calls.append(q_abs.shape[1])
        return real(q_abs, *a, **k)

    monkeypatch.setattr(kernels, "decode_attention", spy)
    fused = []
    real_mp = kernels.merge_project

    def spy_mp(o_lat, *a, **k):
        fused.append(o_lat.shape[1])
        return real_mp(o_lat, *a, **k)

    monkeypatch.setattr(kernels, "merge_project", spy_mp)
    g = torch.Generator().manual_seed(42 + n_head)
    x = torch.randn(2, 160, dim, generator=g).to(dtype)
    xs = [x.to(gpu)]
    with torch.no_grad():
        close(ours(xs[0], 0), ref(x, 0), dtype)
        for step in range(6):
            xd = torch.randn(2, 1, dim, generator=g).to(dtype)
            xs.append(xd.to(gpu))
            close(ours(xs[-1], 160 + step), ref(xd, 160 + step), dtype)
    torch.cuda.synchronize()
    assert_cache_bits(ours, xs, dtype)
    if n_head == 32 and dtype == torch.bfloat16:
        assert calls == [32] * 7, calls  # one launch per call: the prompt and each decode step
    else:
        assert calls == [16] * (7 * -(-n_head // 16)), calls
    # bf16 decode steps run the fused four-launch step (its merge + read-out
    # launch), fewer than 16 heads padded to 16 with zero heads
    if dtype == torch.bfloat16:
        assert fused == [max(n_head, 16)] * 6, fused
    else:
        assert fused == [], fused


def test_out_of_range_positions_raise(gpu):
    """Positions outside the cache raise, as mla.py:413's slice assignment
    does: at once when they are known on the host (int or CPU tensor); for a
    device tensor the kernels skip the token and flag it, check_cache_errors()
    raises, and so does the next eager call once the flag has been read back.
    A no-cache call of a bf16 module longer than the RoPE table raises (the
    reference's grown fp32 table makes its attention see mixed dtypes)."""
    say("out-of-range positions")
    dtype = torch.bfloat16
    cfg = MLAConfig(n_embd=256, max_batch_size=2, max_seq_len=64)
    _, ours = make_pair(cfg, 41, dtype, gpu)
    g = torch.Generator().manual_seed(42)
    step = torch.randn(2, 1, 256, generator=g).to(dtype).to(gpu)
    chunk = torch.randn(2, 8, 256, generator=g).to(dtype).to(gpu)
    with torch.no_grad():
        with pytest.raises(ValueError):
            ours(step, 64)
        with pytest.raises(ValueError):
            ours(step, torch.tensor([3, 64], dtype=torch.int32))
        with pytest.raises(ValueError):
            ours(chunk, torch.tensor([-1, 0], dtype=torch.int32))
        ours(step, torch.tensor([3, 5], dtype=torch.int32, device=gpu))
        ours.check_cache_errors()  # in range: nothing flagged
        # one-token step (append folded into the attention launch)
        ours(step, torch.tensor([3, 64], dtype=torch.int32, device=gpu))
        with pytest.raises(RuntimeError):
            ours.check_cache_errors()
        ours.check_cache_errors()  # the flag was cleared
        # multi-token chunk (separate append), negative start
        out = ours(chunk, torch.tensor([-3, 0], dtype=torch.int32, device=gpu))
        assert bool(torch.isfinite(out.float()).all())
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError):  # the next eager call raises
            ours(step, torch.tensor([9, 9], dtype=torch.int32, device=gpu))
        ours.check_cache_errors()
        ours.set_inference_mode(False)
        ours(torch.randn(1, 64, 256, generator=g).to(dtype).to(gpu), 0)
        with pytest.raises(ValueError):
            ours(torch.randn(1, 65, 256, generator=g).to(dtype).to(gpu), 0)


def test_causal_prompt_mask_equals_unmasked(gpu):
    """SWAMLAModel passes triu(full(-inf), 1)[:T, :T] with every prompt
    (swa_mla_model.py:207-211, :384-387): accepted at start_pos 0 and
    bit-identical to mask=None; any other mask (or a start_pos > 0) raises."""
    say("causal prompt mask")
    dtype = torch.bfloat16
    cfg = MLAConfig(n_embd=512, max_batch_size=2, max_seq_len=96)
    g = torch.Generator().manual_seed(43)
    x = torch.randn(2, 40, 512, generator=g).to(dtype).to(gpu)
    step = torch.randn(2, 1, 512, generator=g).to(dtype).to(gpu)
    mask = torch.triu(torch.full((40, 40), float("-inf")), diagonal=1).to(gpu)
    outs = []
    for use_mask in (False, True):
        _, ours = make_pair(cfg, 44, dtype, gpu)
        with torch.no_grad():
            outs.append((ours(x, 0, None, mask if use_mask else None), ours(step, 40)))
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    _, ours = make_pair(cfg, 44, dtype, gpu)
    with torch.no_grad():
        bad = mask.clone()
        bad[5, 3] = float("-inf")
        with pytest.raises(NotImplementedError):
            ours(x, 0, None, bad)
        with pytest.raises(NotImplementedError):
            ours(x[:, :8], 40, None, mask[:8, :8])
        ours.set_inference_mode(False)  # no cache: the call's own tokens, causal
        ref = ours(x, 0)
        assert torch.equal(ours(x, 0, None, mask), ref)
