"""setuptools entry of the name-only flash_attn distribution (metadata in setup.cfg)."""
from setuptools import setup

setup()
