"""Placeholder for scattermoe.utils.

The reference's scattermoe/utils/replace_moe.py monkey-patches Hugging Face
GptOss/GraniteMoe expert modules at import time; those model families are not
part of this MoE-layer hot path, so nothing is patched here.
"""
