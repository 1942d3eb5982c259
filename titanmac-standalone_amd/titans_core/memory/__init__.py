"""Titans neural long-term memory (memory/neural_memory.py of the reference)."""
from .neural_memory import DecayGate, DeepMemoryMLP, ForgetGate, NeuralMemory

__all__ = ["NeuralMemory", "ForgetGate", "DecayGate", "DeepMemoryMLP"]
