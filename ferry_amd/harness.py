"""End-to-end generation timing on one GPU: greedy decoding with a KV cache, and the serving
metrics the reference reports.

Reference: scripts/run_cell.py:48-76 (``generate``: greedy steps from a common release time,
one device synchronisation and timestamp per generated token) and :147-156 with README.md:
127-138 (the metrics).  With one GPU there is no barrier or broadcast: the release time is
taken after the device has drained.  Metrics of a run of ``steps`` output tokens for
``requests`` sequences:
  TTFT = first token - release;  TPOT = (last token - first token) / (steps - 1);
  E2E = last token - release;    TPS = requests * steps / E2E.

``run_repeats`` is the reference's measurement protocol around ``generate`` (run_cell.py:
124-158): one warm-up run on the warm-up requests, ``discard`` unreported runs on the target
requests, then ``repeats`` measured runs on them, each from an empty expert cache
(``rt.reset()``) and a release time ``release_delay_s`` after the call, with a record per run
(metrics, fetch counts, H2D copies, serial wait, exchange bytes, peak device memory).
``summarize`` reports the measured runs as mean and sample standard deviation
(README.md:136, scripts/summarize.py:13-16).

``synthetic_model`` builds a randomly initialised HF causal LM of a given config with its
dense weights on the GPU and no routed-expert tensors (those live in the pinned pool), the
model the bench runs when no checkpoint is available.
"""
import statistics
import time

import torch

# The reference releases every run 200 ms after its rank 0 reads the clock (run_cell.py:54-55).
RELEASE_DELAY_S = 0.2
METRICS = ('TTFT', 'TPOT', 'E2E', 'TPS')


def _sync(device):
    if device.type == 'cuda':
        torch.cuda.synchronize(device)


def generate(model, input_ids, steps, start_delay_s=0.0):
    """Greedy decoding of ``steps`` tokens after the prompt ``input_ids`` [B, P] (all the same
    length).  Returns dict(release_ns, first_ns, end_ns, step_ns, tokens [B][steps])."""
    dev = input_ids.device
    batch = input_ids.shape[0]
    _sync(dev)
    release = time.perf_counter_ns() + int(start_delay_s * 1e9)
    while time.perf_counter_ns() < release:
        time.sleep(1e-4)
    cache, feed, seen = None, input_ids, 0
    stamps, tokens = [], []
    with torch.inference_mode():
        for _ in range(steps):
            n = feed.shape[1]
            positions = torch.arange(seen, seen + n, device=dev).expand(batch, n)
            mask = torch.ones((batch, seen + n), dtype=torch.long, device=dev)
            out = model(input_ids=feed, attention_mask=mask, position_ids=positions,
                        past_key_values=cache, use_cache=True, logits_to_keep=1)
            cache = out.past_key_values
            nxt = out.logits[:, -1].argmax(-1)
            tokens.append(nxt)
            _sync(dev)
            stamps.append(time.perf_counter_ns())
            seen += n
            feed = nxt[:, None]
    return dict(release_ns=release, first_ns=stamps[0], end_ns=stamps[-1], step_ns=stamps,
                tokens=torch.stack(tokens, 1).cpu().tolist())


def serving_metrics(result, requests, steps):
    """TTFT / TPOT / E2E in seconds and TPS in tokens/s of one ``generate`` result
    (run_cell.py:150-154 at world = 1).  TPOT of a one-token run is 0 (the reference divides
    by steps - 1 = 0 there)."""
    e2e = (result['end_ns'] - result['release_ns']) / 1e9
    ttft = (result['first_ns'] - result['release_ns']) / 1e9
    tpot = (result['end_ns'] - result['first_ns']) / 1e9 / (steps - 1) if steps > 1 else 0.0
    return dict(TTFT=ttft, TPOT=tpot, E2E=e2e, TPS=requests * steps / e2e)


def run_repeats(model, rt, warmup_ids, target_ids, steps, repeats=3, discard=1,
                release_delay_s=RELEASE_DELAY_S, log=None):
    """The reference's repeat protocol on one GPU (run_cell.py:124-158): run 0 is the warm-up
    on ``warmup_ids``, the next ``discard`` runs repeat ``target_ids`` unreported, then
    ``repeats`` measured runs on ``target_ids``.  Every run starts from an empty expert cache
    and history (``rt.reset()``) with the device's peak-memory counter reset, and ``rt.h2d`` is
    drained after it.  Returns one record per run: repeat, phase ('warmup' | 'discard' |
    'target'), TTFT / TPOT / E2E / TPS, the release / first / end timestamps (ns),
    requests, output_tokens, the runtime's counters
    (fetches_per_rank, decode_fetches_per_rank, h2d_copies, serial_wait_s, dispatch_bytes,
    combine_bytes), peak_allocated_bytes and the generated tokens.  ``log`` (optional) is
    called with each record as it completes."""
    if repeats < 1 or discard < 0:
        raise ValueError('repeats must be >= 1 and discard >= 0')
    dev = target_ids.device
    records = []
    for repeat in range(1 + discard + repeats):
        phase = 'warmup' if repeat == 0 else 'discard' if repeat <= discard else 'target'
        ids = warmup_ids if repeat == 0 else target_ids
        rt.reset()
        if dev.type == 'cuda':
            torch.cuda.reset_peak_memory_stats(dev)
        result = generate(model, ids, steps, start_delay_s=release_delay_s)
        rt.h2d.synchronize()
        row = dict(repeat=repeat, phase=phase, **serving_metrics(result, len(ids), steps),
                   release_ns=result['release_ns'], first_ns=result['first_ns'],
                   end_ns=result['end_ns'],
                   requests=len(ids), output_tokens=steps,
                   fetches_per_rank=[int(v) for v in rt.fetches_per_rank],
                   decode_fetches_per_rank=[int(v) for v in rt.decode_fetches_per_rank],
                   h2d_copies=int(rt.h2d.copies), serial_wait_s=rt.serial_wait_ns / 1e9,
                   dispatch_bytes=int(rt.transport.dispatch_bytes),
                   combine_bytes=int(rt.transport.combine_bytes),
                   peak_allocated_bytes=(int(torch.cuda.max_memory_allocated(dev))
                                         if dev.type == 'cuda' else None),
                   tokens=result['tokens'])
        records.append(row)
        if log is not None:
            log(row)
    return records


def summarize(records):
    """Mean and sample standard deviation (0 for one run) of each metric over the measured
    ('target') runs, and the run count (README.md:136, scripts/summarize.py:13-16)."""
    target = [r for r in records if r['phase'] == 'target']
    if not target:
        raise ValueError('no measured runs')
    out = dict(n=len(target))
    for key in METRICS:
        values = [r[key] for r in target]
        out[key] = dict(mean=statistics.mean(values),
                        std=statistics.stdev(values) if len(values) > 1 else 0.0)
    return out


def synthetic_model(config, spec, device='cuda', seed=0, std=0.02):
    """Random-weight HF causal LM of ``config`` on ``device`` (bf16, eval, SDPA attention)
    without its routed-expert tensors: weights ~ N(0, std), norm scales 1."""
    from accelerate import init_empty_weights
    from transformers import AutoModelForCausalLM
    config._attn_implementation = 'sdpa'
    with init_empty_weights(include_buffers=False):
        model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16)
    for index in spec.moe_layers:
        model.model.layers[index].mlp.experts = None
    from .loader import place_buffers, resolve_device
    device = resolve_device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    for name, param in list(model.named_parameters()):
        owner_name, _, attr = name.rpartition('.')
        owner = model.get_submodule(owner_name)
        if 'norm' in attr or 'norm' in owner_name.rsplit('.', 1)[-1]:
            value = torch.ones(param.shape, dtype=torch.bfloat16, device=device)
        else:
            value = (torch.randn(param.shape, generator=gen, device=device) * std).to(torch.bfloat16)
        owner._parameters[attr] = torch.nn.Parameter(value, requires_grad=False)
    if getattr(config, 'tie_word_embeddings', False):
        model.tie_weights()
    place_buffers(model, device)
    return model.eval()
