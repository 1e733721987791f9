"""DeepSeek-V2-Lite q_len=1 decode on the HIP kernels, graph-replayed (reference:
src/run.py; same flags, same JSON report, same TPS definition).

    python flash-deepseek-v2-lite_amd/src/run.py --kernel-family small|batch \
        [--model-path DIR [--prompt TEXT]] \
        [--batch-size B | --batch-sizes "1 64 256"] [--max-new-tokens 100] \
        [--prompt-len 24 | --prompt-len-range LO HI] [--config 1|2|3] \
        [--dump-token-ids] [--dump-step-trace] [--json-out FILE]

With ``--model-path`` (a local DeepSeek-V2-Lite(-Chat) directory: config.json, safetensors
shards, tokenizer files) the weights come from the checkpoint and the prompt is ``--prompt``
through the tokenizer's chat template with the generation prompt, replicated across the
batch -- the reference's run (run.py:14, 719-741; default prompt "Write me a 500 word
novel.").  Without it (there is no checkpoint on these machines) the model is the seeded
random-init DeepSeek-V2-Lite (N(0,0.02) bf16, seed --seed) and the prompt ``--prompt-len``
uniform random token ids (seed --prompt-seed), one prompt replicated across the batch as in
the reference unless ``--prompt-len-range`` draws one length (and prompt) per row.
``--config N`` selects benchmark config N (1: bsz=1 prompt 128 small; 2: bsz=64 lengths
U[256,1024] batch; 3: bsz=256 prompt 2048 batch, one prompt per row).

Beside the reference's JSON fields the report carries hbm_bytes_per_step (the algorithmic
bytes of one step, dsv2lite.roofline), roofline_fraction (those bytes / the mean step time /
8 TB/s) and kernels_per_step (kernel nodes of the captured step).

Flow per batch size (run.py:591-688): prefill -> snapshot -> 3 eager warmup
steps (each followed by a restore) -> capture one step into a hipGraph ->
restore -> ``max_new_tokens - 1`` replays, timed.  TPS = B * (max_new_tokens - 1)
/ decode seconds (run.py:684-686, 698).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

import torch  # noqa: E402

DEFAULT_MAX_NEW_TOKENS = 100
DEFAULT_PROMPT = "Write me a 500 word novel."
DEFAULT_PROMPT_LEN = 24  # length of the reference's chat-templated default prompt
GRAPH_WARMUP_STEPS = 3
PATH_NAMES = {"small": "hip_small_gemv_graph", "batch": "hip_batching_graph"}
CONFIG_PRESETS = {
    1: dict(batch_sizes=[1], kernel_family="small", prompt_len=128, prompt_len_range=None, prompt_seed=1,
            replicate=True),
    2: dict(batch_sizes=[64], kernel_family="batch", prompt_len=None, prompt_len_range=(256, 1024), prompt_seed=2,
            replicate=False),
    3: dict(batch_sizes=[256], kernel_family="batch", prompt_len=2048, prompt_len_range=None, prompt_seed=2,
            replicate=False),
}


def set_kernel_family(kernel_family: str) -> str:
    """Validate a family name (run.py:53-57)."""
    if kernel_family not in PATH_NAMES:
        raise ValueError(f"Unknown kernel family: {kernel_family}")
    return kernel_family


def parse_args(argv: list[str] | None = None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="DeepSeek-V2-Lite decode using a selectable HIP kernel family.")
    p.add_argument("--model-path", type=str, default=None,
                   help="local checkpoint directory (config.json, *.safetensors, tokenizer); random-init weights "
                        "without it")
    p.add_argument("--prompt", type=str, default=DEFAULT_PROMPT, help="user prompt (with --model-path)")
    p.add_argument("--max-new-tokens", type=int, default=DEFAULT_MAX_NEW_TOKENS)
    p.add_argument("--batch-size", type=int, default=1)
    p.add_argument("--batch-sizes", type=str, default=None, help='Comma/space separated sweep, e.g. "1 2 4".')
    p.add_argument("--kernel-family", choices=tuple(PATH_NAMES), default="batch")
    p.add_argument("--device", type=str, default="cuda")
    p.add_argument("--dump-token-ids", action="store_true")
    p.add_argument("--dump-step-trace", action="store_true")
    p.add_argument("--prompt-len", type=int, default=DEFAULT_PROMPT_LEN)
    p.add_argument("--prompt-len-range", type=int, nargs=2, default=None, metavar=("LO", "HI"))
    p.add_argument("--config", type=int, choices=sorted(CONFIG_PRESETS), default=None)
    p.add_argument("--seed", type=int, default=0, help="weight init seed")
    p.add_argument("--prompt-seed", type=int, default=1)
    p.add_argument("--layers", type=int, default=None, help="fewer layers (tests only)")
    p.add_argument("--json-out", type=str, default=None)
    a = p.parse_args(argv)
    a.replicate = a.prompt_len_range is None
    if a.config is not None:
        for k, v in CONFIG_PRESETS[a.config].items():
            setattr(a, k, v)
    return a


def parse_batch_sizes(args: argparse.Namespace) -> list[int]:
    """run.py:239-249: a single size or a sweep; every size and max_new_tokens positive."""
    if isinstance(getattr(args, "batch_sizes", None), list):
        sizes = list(args.batch_sizes)
    elif args.batch_sizes is None:
        sizes = [args.batch_size]
    else:
        sizes = [int(s) for s in args.batch_sizes.replace(",", " ").replace("，", " ").split()]
    if not sizes or any(s <= 0 for s in sizes):
        raise ValueError("batch size must be positive")
    if args.max_new_tokens <= 0:
        raise ValueError("max_new_tokens must be positive")
    return sizes


def make_prompts(args: argparse.Namespace, batch_size: int, vocab: int) -> list[torch.Tensor]:
    g = torch.Generator().manual_seed(args.prompt_seed)
    if args.prompt_len_range is not None:
        lo, hi = args.prompt_len_range
        if not 1 <= lo <= hi:
            raise ValueError("--prompt-len-range needs 1 <= LO <= HI")
        lens = torch.randint(lo, hi + 1, (batch_size,), generator=g).tolist()
        return [torch.randint(0, vocab, (n,), generator=g) for n in lens]
    if args.prompt_len <= 0:
        raise ValueError("prompt length must be positive")
    if not getattr(args, "replicate", True):  # one prompt per row (benchmark config 3)
        return [torch.randint(0, vocab, (args.prompt_len,), generator=g) for _ in range(batch_size)]
    one = torch.randint(0, vocab, (args.prompt_len,), generator=g)
    return [one.clone() for _ in range(batch_size)]


def run_graph_decode(weights, prompts: list[torch.Tensor], family: str, max_new_tokens: int, device,
                     dump_token_ids: bool = False, dump_step_trace: bool = False) -> dict:
    import dsv2lite
    from dsv2lite.roofline import step_bytes

    B = len(prompts)
    lens = [int(p.numel()) for p in prompts]
    eng = dsv2lite.DecodeEngine(weights, [n + max_new_tokens + 8 for n in lens], family=family, device=device)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    first = eng.prefill([p.to(device) for p in prompts]).clone()
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    snap = eng.snapshot()
    rec: list = []
    eng.step(record=rec)  # the routed experts each layer hits, for the byte count of a step
    n_exp = [int(torch.unique(r[2]).numel()) for r in rec if r[0] == "router"]
    del rec
    eng.restore(snap)
    collect = dump_token_ids or dump_step_trace
    gen = [[t] for t in first.cpu().tolist()] if collect else None
    trace = []
    if collect and dump_step_trace:
        trace.append(_trace_entry(0, [r[0] for r in gen], lens))
    for _ in range(GRAPH_WARMUP_STEPS):
        eng.step()
        torch.cuda.synchronize()
        eng.restore(snap)
    eng.capture()
    eng.restore(snap)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for step in range(1, max_new_tokens):
        eng.replay()
        if collect:
            ids = eng.ids.cpu().tolist()
            for r, t in enumerate(ids):
                gen[r].append(t)
            if dump_step_trace:
                trace.append(_trace_entry(step, ids, [n + step for n in lens]))
    torch.cuda.synchronize()
    decode_s = time.perf_counter() - t0
    eng.check_errors()
    out_ids = gen[0] if (gen is not None and B == 1) else gen
    steps = max(max_new_tokens - 1, 0)
    nbytes = step_bytes(eng.cfg, n_exp, sum(n + 1 + (steps - 1) / 2 for n in lens), B)
    return {"batch_size": B, "path": PATH_NAMES[family], "generated_ids": out_ids,
            "decode_tokens": B * steps, "prefill_seconds": prefill_s,
            "decode_seconds": decode_s, "step_trace": trace, "prompt_lens": lens, "hbm_bytes_per_step": nbytes,
            "kernels_per_step": eng.kernels_per_step, "steps": steps}


def _trace_entry(step: int, ids: list[int], positions: list[int]) -> dict:
    e = {"step": step, "cache_position": positions[0] if len(set(positions)) == 1 else positions}
    if len(ids) == 1:
        e["token_id"] = ids[0]
    else:
        e["token_ids"] = ids
    return e


def build_result(run: dict, include_token_ids: bool, include_step_trace: bool) -> dict:
    """run.py:691-705 plus the prompt lengths."""
    ds, dt = run["decode_seconds"], run["decode_tokens"]
    r = {"batch_size": run["batch_size"], "path": run["path"], "ttft_ms": run["prefill_seconds"] * 1000.0,
         "tps": dt / ds if ds > 0 else 0.0, "decode_tokens": dt,
         "prompt_lens": run["prompt_lens"] if len(set(run["prompt_lens"])) > 1 else run["prompt_lens"][0],
         "hbm_bytes_per_step": run["hbm_bytes_per_step"], "kernels_per_step": run["kernels_per_step"]}
    if ds > 0 and run["steps"] > 0:
        from dsv2lite.roofline import roofline_fraction

        r["roofline_fraction"] = roofline_fraction(run["hbm_bytes_per_step"], ds / run["steps"])
    if include_token_ids:
        r["generated_token_ids"] = run["generated_ids"]
    if include_step_trace:
        r["step_trace"] = run["step_trace"]
    return r


def main(argv: list[str] | None = None) -> dict:
    args = parse_args(argv)
    family = set_kernel_family(args.kernel_family)
    if not torch.cuda.is_available():
        raise RuntimeError("a ROCm GPU is required for this benchmark")
    sizes = parse_batch_sizes(args)
    import dsv2lite
    from src.hardware_info import collect_hardware_info

    dev = torch.device(args.device)
    chat_ids = None
    if args.model_path is not None:
        from dsv2lite.checkpoint import chat_prompt_ids, load_tokenizer, load_weights

        weights = load_weights(args.model_path, device=dev, n_layers=args.layers)
        cfg = weights.cfg
        chat_ids = chat_prompt_ids(load_tokenizer(args.model_path), args.prompt)
    else:
        cfg = dsv2lite.DSV2Config() if args.layers is None else dsv2lite.DSV2Config(n_layers=args.layers)
        weights = dsv2lite.init_weights(cfg, device=dev, seed=args.seed)
    results = []
    for B in sizes:
        # the reference replicates the chat-templated prompt across the batch (run.py:739-741)
        prompts = [chat_ids.clone() for _ in range(B)] if chat_ids is not None else make_prompts(args, B, cfg.vocab)
        run = run_graph_decode(weights, prompts, family, args.max_new_tokens, dev, args.dump_token_ids,
                               args.dump_step_trace)
        results.append(build_result(run, args.dump_token_ids, args.dump_step_trace))
    hw = collect_hardware_info(dev)
    out = dict(results[0], hardware=hw) if len(results) == 1 else {"results": results, "hardware": hw}
    text = json.dumps(out, ensure_ascii=False, indent=2)
    if args.json_out:
        with open(args.json_out, "w") as f:
            f.write(text + "\n")
    print(text)
    return out


if __name__ == "__main__":
    main()
