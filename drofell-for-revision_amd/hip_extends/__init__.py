"""HIP (gfx950) native extensions for the quantized-Linear hot path."""
