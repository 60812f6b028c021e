"""Sabah MoE expert runtime, MI355X build (host side)."""
