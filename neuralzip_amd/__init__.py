"""neuralzip_amd: NeuralZip's on-the-fly exponent-lane decompression on MI355X.

The public surface mirrors the reference package (neuralzip/__init__.py:1-16):
``neuralzip(setup=None, *, device=None)`` patches Hugging Face loading and
saving, and ``neuralzip.setup(model, **options)`` builds a NeuralZipSetup.
``matvec_tokens`` (keyword-only, not in the reference, default 0) turns on
the fused decode-matvec for blocks of at most that many token rows.
"""


class _NeuralZip:
    def __call__(self, setup=None, *, device=None, matvec_tokens=0):
        from neuralzip_amd.gpu.pretrained import enable
        return enable(setup, device=device, matvec_tokens=matvec_tokens)

    def setup(self, model, **options):
        from neuralzip_amd.setup import NeuralZipSetup
        return NeuralZipSetup(**options).build(model)


neuralzip = _NeuralZip()

__all__ = ["neuralzip"]
