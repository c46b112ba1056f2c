"""NativeSchedulerBackend (python/tvara/scheduler.py:186-214) with a prompt
decoded in chunked passes (tvara_sequence_prefill) and the iteration batch
decoded on the GPU in one tvara_sequences_decode call.

The interface, the greedy token choice and the error behaviour are the
reference's: keys are served in order, a key whose pending logits are not
finite raises ValueError("Nonfinite model logits") after every key before it
was decoded, and a failing decode leaves the keys (or prompt tokens) before it
decoded.  The batched calls are all-or-nothing, so a failed call is replayed
token by token to reach exactly that state (and that outcome: a replay that
completes is a success).  A key listed twice is decoded twice, the second
time from the logits of the first.
"""

from __future__ import annotations

import numpy as np


class NativeSchedulerBackend:
    def __init__(self, model):
        self.model = model
        self.sequences = {}
        self.pending = {}

    def create(self, key):
        self.sequences[key] = self.model._new_sequence()

    def prefill(self, key, tokens):
        tokens = list(tokens)
        if not tokens:
            return
        try:
            self.pending[key] = self.model.prefill(self.sequences[key], tokens)
        except Exception:
            # nothing was decoded: replay one by one for the reference's partial state
            for token in tokens:
                self.pending[key] = self.model.logits(self.sequences[key], token)

    def _decode_run(self, keys, tokens):
        try:
            out = self.model.decode_sequences([self.sequences[k] for k in keys], tokens)
        except Exception:
            # nothing was decoded: replay one by one for the reference's partial state
            for key, token in zip(keys, tokens):
                self.pending[key] = self.model.logits(self.sequences[key], token)
            return
        for i, key in enumerate(keys):
            self.pending[key] = out[i]

    def decode_batch(self, keys):
        result = []
        run, run_tokens = [], []
        for key in keys:
            if key in run:  # a repeated key starts a new run after the current one is decoded
                self._decode_run(run, run_tokens)
                run, run_tokens = [], []
            logits = self.pending[key]
            if not np.isfinite(logits).all():
                if run:
                    self._decode_run(run, run_tokens)
                raise ValueError("Nonfinite model logits")
            token = int(logits.argmax())
            result.append(token)
            run.append(key)
            run_tokens.append(token)
        if run:
            self._decode_run(run, run_tokens)
        return result

    def drop(self, key):
        self.model._drop_sequence(self.sequences.pop(key))
        self.pending.pop(key, None)
