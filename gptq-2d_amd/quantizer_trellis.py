"""Trellis (QTIP bitshift) quantizer plug-ins -- placeholder until the HIP Viterbi lands."""
