"""MI355X-native codec/vocoder decode stage: HIP kernels for gfx950 behind a C ABI
(``libomni_codec.so``), with host modules that keep the reference vocoder stage's API."""

__version__ = "0.1.0"
