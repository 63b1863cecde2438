"""CPU oracle for the decoder KV-cache hot path — TEST INFRASTRUCTURE ONLY.

A plain numpy restatement of the reference engine's arithmetic on this path,
written from the reference's source text (file:line cited per function):

    oracle.paged_kv   slot mapping, paged append, block-table gather, softmax
                      attention (length-masked and padded/masked forms), paged
                      attention = gather + attention.
    oracle.decoder    the synthetic Whisper-class decoder (DecoderLayer.forward,
                      decode_step, greedy decoding) used for token parity.
    oracle.tts        the streaming multi-codebook TTS model (codebook embedding
                      sum, decoder layers, per-codebook heads, frame-by-frame
                      greedy generation) and the TTS engine's block bookkeeping.
    oracle.cpu_path   the reference's eager CPU path restated in float32 torch
                      (decoder, batched eager decode loop with the pool write,
                      one-layer paged attention step, TTS engine step): the CPU
                      baseline bench.py times on the host cores.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import
anything from this package, and only to check results (or, in bench.py, as the
timed CPU baseline). The product path (speech_serving) never imports it.

Pinning: every oracle function is checked (tests/test_oracle.py,
tests/test_tts_oracle.py, tests/test_cpu_path.py) against closed forms,
invariants, brute force on tiny inputs, the float64 oracle (for cpu_path) and
(for the decoders and the TTS model) golden vectors in tests/golden/.
See each test for which function it pins.
"""
