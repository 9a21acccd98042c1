"""The HIP decode driver (sunnynet_amd/cli.py): the reference CLI's
``decode_stream`` loop (sunnynet/cli.py:57-106) with ``--backend hip``.

CPU: the byte fallback tokenizer (cli.py:224-225), the sampler's filters, and
argument checks. GPU: greedy decoding through ``main`` equals the reference
C runtime's own greedy chain (sn_prefill, then sn_step per token) token for
token, and the statistics carry the reference's keys.
"""
from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from sunnynet_amd.cli import ByteTokenizer, main, sample


def test_byte_fallback_round_trip():
    tk = ByteTokenizer()
    ids = tk.encode("abé")
    assert ids == [1, ord("a") + 2, ord("b") + 2, 0xC3 + 2, 0xA9 + 2]
    assert tk.decode(ids) == "abé"


def test_sampler_filters():
    z = torch.tensor([0.0, 3.0, 1.0, 2.0])
    assert sample(z, 0.0, 0, 1.0) == 1                      # greedy
    torch.manual_seed(0)
    assert {sample(z, 1.0, 1, 1.0) for _ in range(20)} == {1}   # top-1
    torch.manual_seed(0)
    got = {sample(z, 1.0, 2, 1.0) for _ in range(200)}          # top-2: {1, 3}
    assert got == {1, 3}
    # top-p: p(1) = e^3 / (1 + e + e^2 + e^3) = 0.644 > 0.5 -> only token 1
    torch.manual_seed(0)
    assert {sample(z, 1.0, 0, 0.5) for _ in range(50)} == {1}
    # top-p 0.8: tokens 1 (0.644) then 3 (0.237): the mass before 3 is 0.644 < 0.8
    torch.manual_seed(0)
    assert {sample(z, 1.0, 0, 0.8) for _ in range(300)} == {1, 3}
    torch.manual_seed(5)
    a = [sample(z, 0.7, 3, 0.9) for _ in range(10)]
    torch.manual_seed(5)
    assert a == [sample(z, 0.7, 3, 0.9) for _ in range(10)]


def test_rejects_prompt_outside_vocabulary(tmp_path):
    with pytest.raises(SystemExit):
        main(["--blob", str(tmp_path / "none.bin"), "--config", "tiny", "--prompt-ids", "1,999999"])


@pytest.mark.gpu
def test_greedy_cli_matches_reference_runtime(gpu, tmp_path, capsys, ref_built):
    import oracle
    from sunnynet_amd.blob import pack_sunny_blob
    from sunnynet_amd.config import SMALL
    from sunnynet_amd.weights import init_sunnynet

    c = SMALL
    p = tmp_path / "small.bin"
    p.write_bytes(pack_sunny_blob(init_sunnynet(c, 0)))
    prompt = np.random.default_rng(3).integers(0, c.vocab_size, 24).tolist()
    print("cli --backend hip: SunnyNet small, 24-token prompt, 32 greedy tokens", flush=True)
    assert main(["--backend", "hip", "--blob", str(p), "--config", "small", "--prompt-ids",
                 ",".join(map(str, prompt)), "--max-new", "32", "--temperature", "0", "--json"]) == 0
    res = json.loads(capsys.readouterr().out.strip().splitlines()[-1])
    ids = res["ids"]
    assert ids[:24] == prompt and len(ids) == 24 + 32
    assert set(res["stats"]) >= {"prefill_tokens", "prefill_ms", "backend", "gen_tokens",
                                 "decode_ms_median", "decode_ms_per_token"}
    assert res["stats"]["backend"] == "hip" and res["stats"]["gen_tokens"] == 32
    ref = oracle.RefSnModel(p, c.vocab_size, c.dim, c.inner, c.rank, c.taps, c.layers)
    lg = ref.prefill(prompt)
    want = []
    for _ in range(32):
        t = int(np.argmax(lg))
        want.append(t)
        lg = ref.step(t)
    ref.close()
    assert ids[24:] == want
