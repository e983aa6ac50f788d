"""Derive the 32-entry 2^(i/32) table used by the device expf.

tab[i] = bits(double(2^(i/32))) - (i << 47), i.e. the correctly rounded double
of 2^(i/32) with the exponent contribution i/32 * 2^52 removed, so that adding
ki << 47 for any integer ki restores the scaled power of two.  2^(i/32) is
evaluated with 60 significant decimal digits and rounded to double by Python's
correctly rounded Decimal -> float conversion.  Prints C initialisers.
"""
import struct
from decimal import Decimal, getcontext

getcontext().prec = 60
LN2 = Decimal(2).ln()
for i in range(32):
    v = float((LN2 * Decimal(i) / Decimal(32)).exp())
    bits = struct.unpack("<Q", struct.pack("<d", v))[0]
    print("0x%016xULL," % ((bits - (i << 47)) & 0xFFFFFFFFFFFFFFFF))
