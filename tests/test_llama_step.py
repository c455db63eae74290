"""Config 5: a Llama-3.2-1B-shaped decode step (16 layers, hidden 2048, 32/8 heads of 64,
B=32, ctx 2048, bf16 paged KV, random weights; and again over fp8 E4M3 caches) through
the HIP cache write (RoPE fused) and decode attention, against the CPU fp32 oracle: every layer's attention output on the
same inputs (max-abs <= 1e-2, the north star's bar), and top-5 next-token agreement of the
whole step with an fp32 CPU run of the same model."""
import pytest
import torch

import llama_step as L

pytestmark = pytest.mark.gpu


def test_llama_1b_shaped_decode_step():
    cfg = L.Cfg()
    inv = L.llama3_inv_freq(cfg)
    print("[case] config 5 model + cache", flush=True)
    model = L.make_model(cfg, seed=0)
    caches, indptr, ids, last = L.make_cache(cfg, seed=1)
    g = torch.Generator(device="cpu")
    g.manual_seed(2)
    tokens = torch.randint(0, cfg.vocab, (cfg.batch,), generator=g).cuda()
    print("[case] config 5 gpu step", flush=True)
    logits_gpu, errs = L.gpu_step(cfg, model, caches, indptr, ids, last, tokens, inv,
                                  check_rows=range(0, cfg.batch, 4))
    torch.cuda.synchronize()
    print("[case] config 5 cpu step", flush=True)
    logits_cpu = L.cpu_step(cfg, model, caches, indptr, ids, last, tokens, inv)
    overlap, top1 = L.top5_agreement(logits_gpu, logits_cpu)
    print(f"config5 per-layer max-abs attention error: {[f'{e:.2e}' for e in errs]}; "
          f"top-5 overlap {overlap:.3f}, top-1 agreement {top1:.3f}", flush=True)
    assert len(errs) == cfg.layers and max(errs) <= 1e-2
    assert torch.isfinite(logits_gpu).all()
    # bf16 GPU step vs fp32 CPU step: the same next-token candidates
    assert overlap >= 0.8 and top1 >= 0.8


def test_llama_1b_shaped_decode_step_fp8_cache():
    # the same step over fp8 (E4M3) caches, K and V scale 1/16: the history is quantised
    # once, the new token goes through the quantising append; the CPU run quantises it the
    # same way and attends over the dequantised cache
    cfg = L.Cfg()
    inv = L.llama3_inv_freq(cfg)
    scale = 0.0625
    print("[case] config 5 fp8 model + cache", flush=True)
    model = L.make_model(cfg, seed=0)
    caches, indptr, ids, last = L.make_cache(cfg, seed=1, kv_scale=scale)
    g = torch.Generator(device="cpu")
    g.manual_seed(2)
    tokens = torch.randint(0, cfg.vocab, (cfg.batch,), generator=g).cuda()
    print("[case] config 5 fp8 gpu step", flush=True)
    logits_gpu, errs = L.gpu_step(cfg, model, caches, indptr, ids, last, tokens, inv,
                                  check_rows=range(0, cfg.batch, 4), kv_scale=scale)
    torch.cuda.synchronize()
    print("[case] config 5 fp8 cpu step", flush=True)
    logits_cpu = L.cpu_step(cfg, model, caches, indptr, ids, last, tokens, inv, kv_scale=scale)
    overlap, top1 = L.top5_agreement(logits_gpu, logits_cpu)
    print(f"config5 fp8 per-layer max-abs attention error: {[f'{e:.2e}' for e in errs]}; "
          f"top-5 overlap {overlap:.3f}, top-1 agreement {top1:.3f}", flush=True)
    assert len(errs) == cfg.layers and max(errs) <= 1e-2
    assert torch.isfinite(logits_gpu).all()
    assert overlap >= 0.8 and top1 >= 0.8
