"""Writes the golden vectors of the two functions no closed form pins: the draft proposal and the acceptance.

Run once, in the build container where the reference is mounted (never on the GPU box, never from a test):

    TRITON_INTERPRET=1 python tests/golden/make_golden.py /root/reference

It imports the reference package (``src/omniasr_trt``) and its test module (``tests/test_spec.py``) and runs, on
the CPU, the reference's own Triton kernels under Triton's interpreter (``kernels.propose`` -> ``_propose``,
``kernels.accept`` -> ``_accept``) and its PyTorch restatement of the proposal (``reference_propose``), on inputs
drawn as the reference's ``test_propose_kernel`` draws them (B = 8, 2048 positions, vocabularies of 4-8 symbols,
k in {1, 4, 7}) and on random acceptance states.  The two proposal implementations must agree before anything is
written.  Output: ``propose_golden.npz`` and ``accept_golden.npz`` next to this script (inputs and outputs only).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path
from types import SimpleNamespace

import numpy as np

HERE = Path(__file__).resolve().parent


def main(reference: Path) -> None:
    if os.environ.get("TRITON_INTERPRET") != "1":
        raise SystemExit("set TRITON_INTERPRET=1 (the reference's kernels run on the CPU under Triton's interpreter)")
    sys.path.insert(0, str(reference / "src"))
    sys.path.insert(0, str(reference / "tests"))
    import torch
    from omniasr_trt import kernels, llm
    from omniasr_trt.spec import AHEAD, BEHIND, DRAFT_CAPACITY, NGRAM, REACH, SELF_MIN, SELF_WINDOW
    from test_spec import reference_propose

    # ---- proposal: 4 trials for each k, generator of test_propose_kernel (tests/test_spec.py:201-217)
    arrays: dict[str, np.ndarray] = {}
    n = 0
    for k in (1, 4, 7):
        g = torch.Generator().manual_seed(30 + k)
        b, cap = 8, 2048
        for trial in range(4):
            vocab = 4 + trial % 5
            out = torch.randint(3, vocab, (b, cap), dtype=torch.int32, generator=g)
            first = torch.randint(0, 600, (b,), generator=g)
            last = first + torch.randint(0, 1400, (b,), generator=g)
            last[0] = first[0]
            out[torch.arange(cap)[None, :] < first[:, None]] = llm.PAD
            draft = torch.randint(3, vocab, (b, DRAFT_CAPACITY), dtype=torch.int32, generator=g)
            dlen = torch.randint(0, DRAFT_CAPACITY + 1, (b,), generator=g)
            dlen[1] = 0
            draft[torch.arange(DRAFT_CAPACITY)[None, :] >= dlen[:, None]] = -1
            nxt = (torch.rand(b, generator=g) * (dlen + 8)).long()
            st = SimpleNamespace(device=torch.device("cpu"), draft_tokens=k, out=out, draft=draft, draft_len=dlen,
                                 last=last, first=first, next=nxt)
            want, want_draft, want_start = reference_propose(st, b)
            start = torch.empty(b, dtype=torch.long)
            got, got_draft = kernels.propose(out, draft, dlen, last, first, nxt, start, k, NGRAM, BEHIND, AHEAD,
                                             REACH, SELF_WINDOW, SELF_MIN)
            assert torch.equal(got, want) and torch.equal(got_draft, want_draft) and torch.equal(start, want_start), \
                (k, trial)
            p = f"t{n}_"
            arrays.update({p + "k": np.array(k), p + "out": out.numpy(), p + "draft": draft.numpy(),
                           p + "draft_len": dlen.numpy(), p + "last": last.numpy(), p + "first": first.numpy(),
                           p + "next": nxt.numpy(), p + "prop": want.numpy(), p + "use_draft": want_draft.numpy(),
                           p + "start": want_start.numpy()})
            n += 1
    arrays["trials"] = np.array(n)
    arrays["constants"] = np.array([NGRAM, BEHIND, AHEAD, SELF_WINDOW, SELF_MIN] + [x for r in REACH for x in r])
    np.savez_compressed(HERE / "propose_golden.npz", **arrays)
    print(f"propose: {n} trials agree (Triton kernel == PyTorch restatement)")

    # ---- acceptance: random states, fed tokens with planted matches, EOS and the length limit
    g = torch.Generator().manual_seed(7)
    acc: dict[str, np.ndarray] = {}
    cases = 0
    for width in (1, 2, 5, 9):
        for trial in range(6):
            b, cap = 16, 512
            vocab = 3 + trial  # EOS (2) among the argmaxes now and then
            nxt = torch.randint(2, vocab + 3, (b, width), generator=g)
            tokens = torch.randint(2, vocab + 3, (b, width), generator=g)
            agree = torch.rand(b, width, generator=g) < 0.7  # fed token j+1 equal to argmax j, mostly
            tokens[:, 1:] = torch.where(agree[:, 1:], nxt[:, :-1], tokens[:, 1:])
            last = torch.randint(0, cap - 4, (b,), generator=g)
            last[:3] = torch.tensor([cap - 3, cap - 1, 60])  # the clamp at the buffer end, and the limit below
            limit = 62 if trial % 2 else 8188
            done = torch.rand(b, generator=g) < 0.2
            out = torch.full((b, cap), llm.PAD, dtype=torch.int32)  # the writes stand out (and compress)
            tok = tokens[:, 0].clone()
            draft_next = torch.randint(0, 900, (b,), generator=g)
            start = torch.randint(0, 900, (b,), generator=g)
            use_draft = torch.rand(b, generator=g) < 0.5
            before = dict(tokens=tokens.numpy().copy(), nxt=nxt.numpy().copy(), out=out.numpy().copy(),
                          tok=tok.numpy().copy(), last=last.numpy().copy(), done=done.numpy().copy(),
                          draft_next=draft_next.numpy().copy(), start=start.numpy().copy(),
                          use_draft=use_draft.numpy().copy(), limit=np.array(limit), eos=np.array(llm.EOS))
            kernels.accept(tokens, nxt, out, tok, last, done, draft_next, start, use_draft, limit, llm.EOS)
            p = f"c{cases}_"
            acc.update({p + key: v for key, v in before.items()})
            acc.update({p + "out_after": out.numpy(), p + "tok_after": tok.numpy(), p + "last_after": last.numpy(),
                        p + "done_after": done.numpy(), p + "draft_next_after": draft_next.numpy()})
            cases += 1
    acc["cases"] = np.array(cases)
    np.savez_compressed(HERE / "accept_golden.npz", **acc)
    print(f"accept: {cases} cases written")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
