"""ssmjs_amd -- MI355X-native Mamba SSM forward path behind the ssmjs session API."""
